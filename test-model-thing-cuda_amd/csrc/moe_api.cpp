// moe_api.cpp -- C ABI and host orchestration of the MI355X MoE block.
//
// Replaces moe_keep_alloc / moe_ws_alloc / moe_forward / moe_backward /
// moe_aux_from of the reference (tmt-cuda/src/moe.cu:294-545). One handle
// owns one device arena sized at creation; forward and backward only enqueue
// kernels on the caller's stream (no allocation, no host synchronisation).
// Errors are returned as codes with a thread-local message instead of the
// reference's print-and-exit (tmt-cuda/src/common.h:26-33).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/tmt_moe.h"
#include "moe_internal.hpp"

using namespace tmt;

// Scratch of tmt_moe_layernorm_backward_noalloc: a file-scope device array,
// so that entry point never allocates. Each GPU the library runs on holds
// its own copy, at its own address, until the process ends. Host code uses
// the per-device address from hipGetSymbolAddress (scratch_on_current_device),
// never the array's name, which is only a host-side stand-in.
constexpr size_t kNoAllocScratchBytes = size_t(4) << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

#define HIP_TRY(call)                                                              \
    do {                                                                           \
        hipError_t err__ = (call);                                                 \
        if (err__ != hipSuccess)                                                   \
            return fail(TMT_MOE_EDEVICE, "%s failed: %s", #call, hipGetErrorString(err__)); \
    } while (0)

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned_to(const void* p, unsigned a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1u)) == 0; }

// Device address of `scratch` on the current device, looked up on the first
// call made with that device current and kept per device.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_addr[kMaxDevices] = {};

int scratch_on_current_device(float** out) {
    int dev = -1;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(TMT_MOE_EINVAL, "device index %d is out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_addr[dev] == nullptr) {
        void* addr = nullptr;
        const hipError_t err = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
        if (err != hipSuccess || addr == nullptr) {
            (void)hipGetLastError();
            return fail(TMT_MOE_EDEVICE, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                        hipGetErrorString(err));
        }
        g_scratch_addr[dev] = static_cast<float*>(addr);
    }
    *out = g_scratch_addr[dev];
    return TMT_MOE_OK;
}

struct Layout {
    size_t total = 0;
    size_t add(size_t bytes) {
        size_t off = total;
        total += (bytes + 255) & ~size_t(255);
        return off;
    }
};

}  // namespace

struct tmt_moe {
    tmt_moe_desc desc;  // the widths the kernels run at (d and hidden rounded up to 64)
    tmt_moe_desc user;  // the caller's descriptor
    // d or hidden not a multiple of 64: every call copies its operands into
    // zero-padded internal buffers of the rounded-up widths and copies the
    // results back (zero rows and columns contribute nothing to any product,
    // so the routing and every result on the caller's columns are unchanged)
    bool padded = false;
    unsigned align_bf16 = 16, align_f32 = 16;  // pointer alignment the checks require
    uint16_t *px = nullptr, *py = nullptr, *pdy = nullptr, *pdx = nullptr, *pwr = nullptr;
    float* pdwr = nullptr;
    uint16_t* pwu[kMaxExperts] = {};
    uint16_t* pwd[kMaxExperts] = {};
    float* pdwu[kMaxExperts] = {};
    float* pdwd[kMaxExperts] = {};
    int hn = 0;        // width of the first expert GEMM (h, or d for h == 0)
    int nblk_max = 0;  // router blocks at the largest T
    int device = 0;
    char* arena = nullptr;      // per-layer state (the reference's MoeKeep)
    size_t arena_bytes = 0;
    char* ws = nullptr;         // transient buffers (the reference's MoeWs): in the
                                // arena, or a caller workspace shared by handles
    bool own_ws = true;
    // routing state (kept from forward for backward; the reference's MoeKeep)
    float *logits, *probs, *lse, *gate, *blkstat, *stats;
    int32_t* ticket = nullptr;  // decode router's completion counter (zero between calls)
    float* split = nullptr;     // split-K partial tiles of GEMM_DOWN / GEMM_DX (nullptr: none)
    float* dpart = nullptr;     // decode GEMM_DOWN: fp32 rows of the two K halves (nullptr: none)
    int resident = 0;           // workgroups the GPU runs at once (one per CU)
    int32_t *idx, *blkcnt, *blkbase, *counts, *offsets, *order, *perm, *slot_of;
    // activations (U: the single linear's output when hidden = 0, silu'(U)
    // when hidden > 0)
    uint16_t *U, *Aact, *O, *dO, *dU, *dXg, *Xg;
    uint16_t* wt = nullptr;  // W_up transposed ([E][d][hn]) for the backward's GEMM_DX (nullptr: none)
    // MX handles: activations of the two expert GEMMs as two MXFP6 terms
    uint8_t *xq = nullptr, *xq_scales = nullptr, *aq = nullptr, *aq_scales = nullptr;
    // and the call's weight codes in K planes: W_up [E][h][d/2], then W_down [E][d][h/2]
    uint8_t* wplanes = nullptr;
    float *dlogits, *dwr_partial;
    // LayerNorm in front of the block (tmt_moe_forward_ln / tmt_moe_backward_ln)
    uint16_t *H, *dH;
    float *ln_mean, *ln_rstd, *ln_partial, *ln_partial2;
    int last_T = -1;
    bool last_ln = false;  // the last forward was tmt_moe_forward_ln
    // per-kernel event timing (tmt_moe_set_profiling)
    bool prof_on = false;
    std::vector<hipEvent_t> prof_events;  // pairs: start, stop
    std::vector<int> prof_phase;          // phase of each recorded pair
    double prof_ms[TMT_MOE_NPHASES] = {};
    int32_t prof_cnt[TMT_MOE_NPHASES] = {};
};

namespace {

int round64(int v) { return (v + 63) / 64 * 64; }

// The widths the kernels run at: bf16 handles round d and hidden up to
// multiples of 64 (the GEMM tiles' K step and the router's lane layout);
// MXFP4 handles take them as given (validate_desc requires multiples of 64).
tmt_moe_desc internal_desc(const tmt_moe_desc& u) {
    tmt_moe_desc d = u;
    if (u.weight_format == TMT_MOE_WEIGHTS_BF16) {
        d.d = round64(u.d);
        d.hidden = u.hidden > 0 ? round64(u.hidden) : 0;
    }
    return d;
}
bool is_padded(const tmt_moe_desc& u) {
    const tmt_moe_desc d = internal_desc(u);
    return d.d != u.d || d.hidden != u.hidden;
}

// The weight formats on the scaled FP6 x FP4 MFMA.
bool is_mx(int fmt) { return fmt == TMT_MOE_WEIGHTS_MXFP4_MX || fmt == TMT_MOE_WEIGHTS_MXFP4_MX_PLANES; }

int validate_desc(const tmt_moe_desc* d) {
    if (!d) return fail(TMT_MOE_EINVAL, "descriptor is NULL");
    if (d->max_tokens < 1) return fail(TMT_MOE_EINVAL, "max_tokens must be >= 1");
    // any width, as TMT's validate_cfg (config.h:46-52): d >= 1
    if (d->d < 1 || d->d > (1 << 20)) return fail(TMT_MOE_EINVAL, "d=%d must be in [1, 2^20]", d->d);
    if (d->experts < 1 || d->experts > kMaxExperts)
        return fail(TMT_MOE_EINVAL, "experts=%d must be in [1, %d]", d->experts, kMaxExperts);
    if (d->topk < 1 || d->topk > d->experts || d->topk > kMaxTopK)
        return fail(TMT_MOE_EINVAL, "require 1 <= topk <= min(experts, %d) (topk=%d)", kMaxTopK, d->topk);
    if (d->hidden < 0 || d->hidden > (1 << 20))
        return fail(TMT_MOE_EINVAL, "hidden=%d must be in [0, 2^20]", d->hidden);
    if ((int64_t)d->max_tokens * d->topk >= (1ll << 31))
        return fail(TMT_MOE_EINVAL, "max_tokens*topk must fit in int32");
    if (d->weight_format != TMT_MOE_WEIGHTS_BF16 && d->weight_format != TMT_MOE_WEIGHTS_MXFP4 &&
        !is_mx(d->weight_format))
        return fail(TMT_MOE_EINVAL, "unknown weight_format %d", d->weight_format);
    if (is_mx(d->weight_format)) {
        // the scaled-MFMA GEMMs address operands with 32-bit byte offsets
        const int64_t TK = (int64_t)d->max_tokens * d->topk;
        const int64_t widest = std::max<int64_t>(d->d, d->hidden);
        if (TK * (widest / 32) * 48 >= (int64_t(1) << 31) || (int64_t)d->hidden * d->d / 2 >= (int64_t(1) << 31))
            return fail(TMT_MOE_EINVAL, "max_tokens*topk=%lld is too large for MX activations at d=%d, hidden=%d",
                        (long long)TK, d->d, d->hidden);
    }
    if (d->weight_format != TMT_MOE_WEIGHTS_BF16 && d->hidden == 0)
        return fail(TMT_MOE_EINVAL, "MXFP4 weights need hidden > 0");
    // the MX blocks of 32 run along d and hidden, and the FP4 GEMMs step K by 64
    if (d->weight_format != TMT_MOE_WEIGHTS_BF16 && (d->d % 64 != 0 || d->hidden % 64 != 0))
        return fail(TMT_MOE_EINVAL, "MXFP4 weights need d and hidden multiples of 64 (d=%d, hidden=%d)", d->d,
                    d->hidden);
    const tmt_moe_desc in = internal_desc(*d);
    if ((int64_t)d->max_tokens * in.d >= (int64_t(1) << 40) || (int64_t)in.hidden * in.d >= (int64_t(1) << 31))
        return fail(TMT_MOE_EINVAL, "d=%d, hidden=%d too large", d->d, d->hidden);
    return TMT_MOE_OK;
}

// Router rows per workgroup: kRouterWaves waves x R rows x iterations, aiming
// at a few hundred workgroups and staying within the permutation kernel's
// group limit.
int router_rows_per_block(int T, int E, int K) {
    const int R = router_rows_per_wave(E);
    const int base = kRouterWaves * R;
    int iter = T / (base * 512);
    const int rg = 64 / K;
    int iter_max = (64 * rg) / base;
    if (iter_max > 16) iter_max = 16;
    if (iter > iter_max) iter = iter_max;
    if (iter < 1) iter = 1;
    return base * iter;
}

// Device memory of one handle, in two parts:
//   layer  -- state kept from forward to backward (routing, offsets,
//             permutation, U / SiLU(U) / O, the LayerNorm output and row
//             statistics): the reference's MoeKeep (moe.cu:294-315);
//   shared -- buffers that live within one call (router block tables, split-K
//             partials, and every backward operand: dO, dU, dXg, Xg, dlogits,
//             router-dW and LayerNorm partials, dH): the reference's MoeWs
//             (moe.cu:316-328), which one set serves for all layers because
//             layers run one after another (model.cu:104, 254).
struct Sizes {
    size_t layer = 0, shared = 0;
};

Sizes plan(const tmt_moe_desc* user, tmt_moe* m) {
    const tmt_moe_desc din = internal_desc(*user);
    const tmt_moe_desc* d = &din;
    const int64_t T = d->max_tokens, E = d->experts, K = d->topk, D = d->d, h = d->hidden;
    const int64_t hn = h > 0 ? h : D;
    const int64_t TK = T * K;
    const int rpb_min = kRouterWaves * router_rows_per_wave((int)E);
    const int64_t nblk = (T + rpb_min - 1) / rpb_min;
    Layout L, W;
    size_t o_logits = L.add(T * E * 4), o_probs = L.add(T * E * 4), o_lse = L.add(T * 4);
    size_t o_gate = L.add(TK * 4), o_idx = L.add(TK * 4);
    size_t o_counts = L.add(E * 4), o_offsets = L.add((E + 1) * 4), o_order = L.add(E * 4);
    size_t o_stats = L.add((2 + E) * 4);
    size_t o_ticket = L.add(4);
    size_t o_perm = L.add(TK * 4), o_slot = L.add(TK * 4);
    // MX handles (scaled-MFMA FP4 forward) keep activations in MX6x2 form instead of U / SiLU(U)
    const bool mx = is_mx(d->weight_format);
    // U: the single linear's output (hidden = 0), else silu'(U) for the
    // backward; MXFP4 handles are forward-only and keep neither
    const bool fp4 = d->weight_format != TMT_MOE_WEIGHTS_BF16;
    size_t o_U = fp4 ? 0 : L.add(TK * hn * 2);
    size_t o_A = h > 0 && !mx ? L.add(TK * h * 2) : 0;
    size_t o_O = h > 0 ? L.add(TK * D * 2) : 0;
    size_t o_H = L.add(T * D * 2), o_mean = L.add(T * 4), o_rstd = L.add(T * 4);
    // transient
    size_t o_blkcnt = W.add(nblk * E * 4), o_blkbase = W.add(nblk * E * 4);
    size_t o_blkstat = W.add(nblk * (E + 1) * 4);
    // MXFP4 handles are forward-only: no backward buffers.
    const bool bwd = d->weight_format == TMT_MOE_WEIGHTS_BF16;
    size_t o_dO = bwd ? W.add(TK * D * 2) : 0;
    size_t o_dU = bwd && h > 0 ? W.add(TK * h * 2) : 0;
    size_t o_dXg = bwd ? W.add(TK * D * 2) : 0;
    // W_up transposed to [E][d][hn] for GEMM_DX on 256 x 256 tiles (handles
    // whose largest batch runs it there): the GEMM then reads both operands
    // K-contiguous, as GEMM_DOWN does
    const bool wt = bwd && 2 * ((TK + 255) / 256) * ((D + 255) / 256) >= cu_count();
    size_t o_wt = wt ? W.add(E * hn * D * 2) : 0;
    size_t o_Xg = bwd ? W.add(TK * D * 2) : 0;
    size_t o_dl = bwd ? W.add(T * E * 4) : 0;
    size_t o_dwr = bwd ? W.add((size_t)router_dw_chunks_max((int)T, (int)E, (int)D) * E * D * 4) : 0;
    size_t o_dH = bwd ? W.add(T * D * 2) : 0;
    // Split-K tail of the tiled GEMM_DOWN / GEMM_DX (decode-sized handles never tile).
    const bool split = d->weight_format == TMT_MOE_WEIGHTS_BF16 && T > kSkinnyMaxTokens;
    const int resident = cu_count();
    size_t o_split = split ? W.add(gemm_split_floats(resident) * 4) : 0;
    // Decode GEMM_DOWN in K halves: [2][min(T, 64) * K][d] fp32.
    const bool dsplit = d->weight_format == TMT_MOE_WEIGHTS_BF16 && h > 0;
    size_t o_dpart = dsplit ? W.add((size_t)2 * std::min<int64_t>(T, kSkinnyMaxTokens) * K * D * 4) : 0;
    size_t o_xq = mx ? W.add(mx_codes_bytes(TK, D)) : 0, o_xqs = mx ? W.add(mx_scales_bytes(TK, D)) : 0;
    size_t o_aq = mx ? W.add(mx_codes_bytes(TK, h)) : 0, o_aqs = mx ? W.add(mx_scales_bytes(TK, h)) : 0;
    size_t o_wpl = d->weight_format == TMT_MOE_WEIGHTS_MXFP4_MX ? W.add((size_t)E * h * D) : 0;
    const int64_t ln_rows = std::max(scatter_blocks((int)T), ln_chunks((int)T));
    size_t o_lnp = bwd ? W.add((size_t)ln_rows * 2 * D * 4) : 0;
    size_t o_lnp2 = bwd ? W.add((size_t)colsum_groups((int)ln_rows) * 2 * D * 4) : 0;
    // zero-padded operand copies of a handle whose widths are not multiples
    // of 64 (transient: every call fills the ones it reads)
    const bool pad = is_padded(*user);
    size_t o_px = 0, o_py = 0, o_pdy = 0, o_pdx = 0, o_pwr = 0, o_pdwr = 0;
    size_t o_pwu[kMaxExperts] = {}, o_pwd[kMaxExperts] = {}, o_pdwu[kMaxExperts] = {}, o_pdwd[kMaxExperts] = {};
    if (pad) {
        o_px = W.add(T * D * 2);
        o_py = W.add(T * D * 2);
        o_pdy = W.add(T * D * 2);
        o_pdx = W.add(T * D * 2);
        o_pwr = W.add(E * D * 2);
        o_pdwr = W.add(E * D * 4);
        for (int64_t e = 0; e < E; ++e) {
            o_pwu[e] = W.add(hn * D * 2);
            o_pdwu[e] = W.add(hn * D * 4);
            if (h > 0) {
                o_pwd[e] = W.add(D * h * 2);
                o_pdwd[e] = W.add(D * h * 4);
            }
        }
    }
    if (m) {
        char* a = m->arena;
        char* w = m->ws;
        m->logits = (float*)(a + o_logits);
        m->probs = (float*)(a + o_probs);
        m->lse = (float*)(a + o_lse);
        m->gate = (float*)(a + o_gate);
        m->idx = (int32_t*)(a + o_idx);
        m->blkcnt = (int32_t*)(w + o_blkcnt);
        m->blkbase = (int32_t*)(w + o_blkbase);
        m->blkstat = (float*)(w + o_blkstat);
        m->counts = (int32_t*)(a + o_counts);
        m->offsets = (int32_t*)(a + o_offsets);
        m->order = (int32_t*)(a + o_order);
        m->stats = (float*)(a + o_stats);
        m->ticket = (int32_t*)(a + o_ticket);
        m->split = split ? (float*)(w + o_split) : nullptr;
        m->dpart = dsplit ? (float*)(w + o_dpart) : nullptr;
        m->resident = resident;
        m->perm = (int32_t*)(a + o_perm);
        m->slot_of = (int32_t*)(a + o_slot);
        m->U = fp4 ? nullptr : (uint16_t*)(a + o_U);
        m->Aact = h > 0 && !mx ? (uint16_t*)(a + o_A) : nullptr;
        m->xq = mx ? (uint8_t*)(w + o_xq) : nullptr;
        m->xq_scales = mx ? (uint8_t*)(w + o_xqs) : nullptr;
        m->aq = mx ? (uint8_t*)(w + o_aq) : nullptr;
        m->aq_scales = mx ? (uint8_t*)(w + o_aqs) : nullptr;
        m->wplanes = d->weight_format == TMT_MOE_WEIGHTS_MXFP4_MX ? (uint8_t*)(w + o_wpl) : nullptr;
        m->O = h > 0 ? (uint16_t*)(a + o_O) : nullptr;
        m->dO = bwd ? (uint16_t*)(w + o_dO) : nullptr;
        m->dU = bwd ? (h > 0 ? (uint16_t*)(w + o_dU) : m->dO) : nullptr;  // h == 0: combine_bwd writes dU
        m->dXg = bwd ? (uint16_t*)(w + o_dXg) : nullptr;
        m->wt = wt ? (uint16_t*)(w + o_wt) : nullptr;
        m->Xg = bwd ? (uint16_t*)(w + o_Xg) : nullptr;
        m->dlogits = bwd ? (float*)(w + o_dl) : nullptr;
        m->dwr_partial = bwd ? (float*)(w + o_dwr) : nullptr;
        m->H = (uint16_t*)(a + o_H);
        m->ln_mean = (float*)(a + o_mean);
        m->ln_rstd = (float*)(a + o_rstd);
        m->dH = bwd ? (uint16_t*)(w + o_dH) : nullptr;
        m->ln_partial = bwd ? (float*)(w + o_lnp) : nullptr;
        m->ln_partial2 = bwd ? (float*)(w + o_lnp2) : nullptr;
        m->nblk_max = (int)nblk;
        m->padded = pad;
        if (pad) {
            m->px = (uint16_t*)(w + o_px);
            m->py = (uint16_t*)(w + o_py);
            m->pdy = (uint16_t*)(w + o_pdy);
            m->pdx = (uint16_t*)(w + o_pdx);
            m->pwr = (uint16_t*)(w + o_pwr);
            m->pdwr = (float*)(w + o_pdwr);
            for (int64_t e = 0; e < E; ++e) {
                m->pwu[e] = (uint16_t*)(w + o_pwu[e]);
                m->pdwu[e] = (float*)(w + o_pdwu[e]);
                m->pwd[e] = h > 0 ? (uint16_t*)(w + o_pwd[e]) : nullptr;
                m->pdwd[e] = h > 0 ? (float*)(w + o_pdwd[e]) : nullptr;
            }
        }
    }
    return Sizes{L.total, W.total};
}

int check_device(const tmt_moe* m) {
    int dev = -1;
    HIP_TRY(hipGetDevice(&dev));
    if (dev != m->device)
        return fail(TMT_MOE_EINVAL, "handle was created on device %d but device %d is current", m->device, dev);
    return TMT_MOE_OK;
}

constexpr int kProfPairs = 2048;

// Waits for every recorded pair and folds it into the per-phase totals.
int prof_flush(tmt_moe* m) {
    for (size_t i = 0; i < m->prof_phase.size(); ++i) {
        HIP_TRY(hipEventSynchronize(m->prof_events[2 * i + 1]));
        float ms = 0.0f;
        HIP_TRY(hipEventElapsedTime(&ms, m->prof_events[2 * i], m->prof_events[2 * i + 1]));
        m->prof_ms[m->prof_phase[i]] += ms;
        m->prof_cnt[m->prof_phase[i]] += 1;
    }
    m->prof_phase.clear();
    return TMT_MOE_OK;
}

int prof_begin(tmt_moe* m, int phase, hipStream_t s, int* slot) {
    *slot = -1;
    if (!m->prof_on) return TMT_MOE_OK;
    if ((int)m->prof_phase.size() == kProfPairs) {
        int rc = prof_flush(m);
        if (rc) return rc;
    }
    *slot = (int)m->prof_phase.size();
    m->prof_phase.push_back(phase);
    HIP_TRY(hipEventRecord(m->prof_events[2 * *slot], s));
    return TMT_MOE_OK;
}

int prof_end(tmt_moe* m, int slot, hipStream_t s) {
    if (slot < 0) return TMT_MOE_OK;
    HIP_TRY(hipEventRecord(m->prof_events[2 * slot + 1], s));
    return TMT_MOE_OK;
}

// Launch `call` (returning hipError_t) as phase `ph`, timed when profiling.
#define LAUNCH(ph, call)                                  \
    do {                                                  \
        int slot__ = -1;                                  \
        int rc__ = prof_begin(m, (ph), s, &slot__);       \
        if (rc__) return rc__;                            \
        HIP_TRY(call);                                    \
        rc__ = prof_end(m, slot__, s);                    \
        if (rc__) return rc__;                            \
    } while (0)

// Router, scan and permutation arguments of a decode batch (T <= 64): the
// outputs route_small_kernel writes, or the one-token GEMM_UP that routes its
// token itself.
Route1 small_route_params(tmt_moe* m, int T, const uint16_t* X, const uint16_t* Wr, const float* bias) {
    const int E = m->desc.experts, K = m->desc.topk, d = m->desc.d;
    Route1 r{};
    RouterParams& rp = r.rp;
    rp.X = X; rp.Wr = Wr; rp.bias = bias;
    rp.T = T; rp.d = d; rp.E = E; rp.K = K; rp.rows_per_block = T;
    rp.logits = m->logits; rp.probs = m->probs; rp.idx = m->idx; rp.gate = m->gate;
    rp.lse = m->lse;
    ScanParams& sp = r.sp;
    sp.T = T; sp.E = E; sp.K = K; sp.nblk = 1;
    sp.counts = m->counts; sp.offsets = m->offsets; sp.order = m->order; sp.stats = m->stats;
    PermuteParams& pp = r.pp;
    pp.T = T; pp.E = E; pp.K = K; pp.rows_per_block = T;
    pp.perm = m->perm; pp.slot_of = m->slot_of;
    return r;
}

// Routing + dispatch: router / scan / permute (E > 1) or identity (E == 1).
// picks_only (decode batches whose GEMM_UP runs with self_dispatch): the
// router writes the picks and the GEMM_UP completes the dispatch.
// The LayerNorm that tmt_moe_forward_ln hands to the router (S, gamma, beta).
struct LnFuse {
    const uint16_t* S;
    const float* gamma;
    const float* beta;
};
// Routed batches (E > 1, more than kSmallRouteTokens tokens) whose rows the
// router can normalise itself.
bool ln_in_router(int T, int E, int d) { return E > 1 && T > kSmallRouteTokens && router_ln_fits(E, d); }

// ln: the router computes H = LayerNorm(ln->S) into m->H (with the row
// statistics) and routes H; only where ln_in_router holds.
int route(tmt_moe* m, hipStream_t s, int T, const uint16_t* X, const uint16_t* Wr, const float* bias,
          bool picks_only = false, const LnFuse* ln = nullptr) {
    const int E = m->desc.experts, K = m->desc.topk, d = m->desc.d;
    if (ln && !ln_in_router(T, E, d)) return fail(TMT_MOE_EINVAL, "internal: LayerNorm not fusable into this router");
    if (E == 1) {
        LAUNCH(TMT_MOE_PH_PERMUTE, launch_dense_dispatch(T, m->perm, m->slot_of, m->gate, m->counts,
                                                        m->offsets, m->order, m->stats, s));
        return TMT_MOE_OK;
    }
    if (T >= 1 && T <= kSmallRouteTokens) {
        const Route1 r = small_route_params(m, T, X, Wr, bias);
        LAUNCH(TMT_MOE_PH_ROUTER, launch_route_small(r.rp, r.sp, r.pp, picks_only ? nullptr : m->ticket, s));
        return TMT_MOE_OK;
    }
    // without the LayerNorm the logits come from the matrix cores (with the
    // canonical order for rows whose ranking that could change)
    const bool mfma = ln == nullptr && router_mfma_fits(T, E, K, d);
    const int rpb = mfma ? kMfmaRouterRows : router_rows_per_block(T, E, K);
    const int nblk = T > 0 ? (T + rpb - 1) / rpb : 0;
    if (nblk > m->nblk_max) return fail(TMT_MOE_EINVAL, "internal: router block count %d > %d", nblk, m->nblk_max);
    if (nblk > 0) {
        RouterParams rp{};
        rp.X = X; rp.Wr = Wr; rp.bias = bias;
        rp.T = T; rp.d = d; rp.E = E; rp.K = K; rp.rows_per_block = rpb;
        rp.logits = m->logits; rp.probs = m->probs; rp.idx = m->idx; rp.gate = m->gate;
        rp.lse = m->lse; rp.blkcnt = m->blkcnt; rp.blkstat = m->blkstat;
        if (ln) {
            rp.X = ln->S; rp.ln_gamma = ln->gamma; rp.ln_beta = ln->beta;
            rp.ln_H = m->H; rp.ln_mean = m->ln_mean; rp.ln_rstd = m->ln_rstd;
        }
        LAUNCH(TMT_MOE_PH_ROUTER, mfma ? launch_router_mfma(rp, nblk, s) : launch_router(rp, nblk, s));
    }
    ScanParams sp{};
    sp.blkcnt = m->blkcnt; sp.blkstat = m->blkstat; sp.nblk = nblk; sp.T = T; sp.E = E; sp.K = K;
    sp.counts = m->counts; sp.offsets = m->offsets; sp.blkbase = m->blkbase; sp.order = m->order;
    sp.stats = m->stats;
    PermuteParams pp{};
    pp.idx = m->idx; pp.blkbase = m->blkbase; pp.T = T; pp.E = E; pp.K = K;
    pp.rows_per_block = rpb; pp.perm = m->perm; pp.slot_of = m->slot_of;
    if (nblk > 0 && nblk <= kFusedScanBlocks) {
        // few router blocks: the permutation kernel does the scan itself
        LAUNCH(TMT_MOE_PH_PERMUTE, launch_permute_scan(pp, sp, nblk, s));
        return TMT_MOE_OK;
    }
    LAUNCH(TMT_MOE_PH_SCAN, launch_scan(sp, s));
    if (nblk > 0) LAUNCH(TMT_MOE_PH_PERMUTE, launch_permute(pp, nblk, s));
    return TMT_MOE_OK;
}

int check_ptrs(const void* const* tab, int n, const char* what, unsigned align = 16) {
    if (!tab) return fail(TMT_MOE_EINVAL, "%s table is NULL", what);
    for (int e = 0; e < n; ++e) {
        if (!tab[e]) return fail(TMT_MOE_EINVAL, "%s[%d] is NULL", what, e);
        if (!aligned_to(tab[e], align)) return fail(TMT_MOE_EINVAL, "%s[%d] is not %u-byte aligned", what, e, align);
    }
    return TMT_MOE_OK;
}

// Argument checks of the bf16 forward; `xname` names the tensor the router
// reads (X, or S for the LayerNorm variant).
int check_forward(tmt_moe* m, int T, const uint16_t* X, const char* xname, const uint16_t* Wr,
                  const uint16_t* const* W_up, const uint16_t* const* W_down, const uint16_t* Y) {
    if (!m) return fail(TMT_MOE_EINVAL, "handle is NULL");
    const tmt_moe_desc& ds = m->desc;
    if (ds.weight_format != TMT_MOE_WEIGHTS_BF16)
        return fail(TMT_MOE_EINVAL, "handle expects MXFP4 weights: use tmt_moe_forward_mxfp4");
    if (T < 0 || T > ds.max_tokens) return fail(TMT_MOE_EINVAL, "T=%d outside [0, %d]", T, ds.max_tokens);
    if (T > 0 && (!X || !Y)) return fail(TMT_MOE_EINVAL, "%s and Y must be non-NULL", xname);
    const unsigned a = m->align_bf16;
    if (!aligned_to(X, a) || !aligned_to(Y, a))
        return fail(TMT_MOE_EINVAL, "%s and Y must be %u-byte aligned", xname, a);
    if (ds.experts > 1 && (!Wr || !aligned_to(Wr, a)))
        return fail(TMT_MOE_EINVAL, "Wr must be a %u-byte aligned pointer when experts > 1", a);
    int rc = check_ptrs((const void* const*)W_up, ds.experts, "W_up", a);
    if (rc) return rc;
    if (ds.hidden > 0 && (rc = check_ptrs((const void* const*)W_down, ds.experts, "W_down", a))) return rc;
    return check_device(m);
}

// Routing, expert GEMMs and combine of the bf16 forward (arguments checked).
// ln: the router normalises the block input itself (X is then m->H, which the
// router writes before any expert GEMM reads it).
int run_forward(tmt_moe* m, hipStream_t s, int T, const uint16_t* X, const uint16_t* Wr,
                const float* logit_bias, const uint16_t* const* W_up, const uint16_t* const* W_down,
                uint16_t* Y, float beta, const LnFuse* ln = nullptr) {
    const tmt_moe_desc& ds = m->desc;
    const int E = ds.experts, K = ds.topk, d = ds.d, h = ds.hidden, hn = m->hn;
    int rc;
    m->last_T = -1;

    // Decode-sized batches stream the weights with the skinny kernels. Where
    // every expert GEMM runs on the stream variant, the router writes only
    // the picks and each later kernel finds its rows from the pick table
    // (no cross-block handoff inside the router); the combine's extra
    // workgroup writes the dispatch tables.
    const bool skinny = T <= kSkinnyMaxTokens;
    const bool self = skinny && skinny_self_dispatch(T, E, K, d, h, hn);
    // One token whose down GEMM and combine run as one launch: the up GEMM
    // routes the token itself, so the forward is two launches.
    const bool fused1 = T == 1 && h > 0 && E > 1 && decode1_down_combine_fits(d, h, K);
    const bool route1 = fused1 && skinny_up_route1_fits(d, E);
    if (ln && (route1 || self)) return fail(TMT_MOE_EINVAL, "internal: LayerNorm not fusable into this router");
    if (!route1 && (rc = route(m, s, T, X, Wr, logit_bias, self, ln))) return rc;
    if (T > 0) {
        GemmParams up{};
        up.offsets = m->offsets; up.order = m->order; up.perm = m->perm; up.E = E;
        up.idx = E > 1 ? m->idx : nullptr; up.topk = K;
        up.N = hn; up.K = d; up.slots = T * K;
        up.a = X; up.lda = d; up.c = m->U; up.ldc = hn; up.c2 = m->Aact;
        for (int e = 0; e < E; ++e) up.w[e] = W_up[e];
        up.ldb = d;
        up.self_dispatch = self ? 1 : 0;
        bool halves = false;  // decode GEMM_DOWN wrote fp32 K halves instead of O
        if (route1) {
            const Route1 r = small_route_params(m, T, X, Wr, logit_bias);
            LAUNCH(TMT_MOE_PH_GEMM_UP, launch_skinny_up_route1(true, up, r, s));
        } else {
            LAUNCH(TMT_MOE_PH_GEMM_UP, skinny ? launch_skinny_gemm(GEMM_UP, h > 0, up, T, s)
                                              : launch_gemm(GEMM_UP, h > 0, up, s));
        }
        if (fused1) {
            Down1Params dp{};
            for (int e = 0; e < E; ++e) dp.w[e] = W_down[e];
            dp.a = m->Aact; dp.idx = m->idx; dp.gate = m->gate; dp.slot_of = m->slot_of;
            dp.O = m->O; dp.Y = Y; dp.beta = beta; dp.d = d; dp.h = h; dp.K = K;
            LAUNCH(TMT_MOE_PH_GEMM_DOWN, launch_decode1_down_combine(dp, s));
            m->last_T = T;
            return TMT_MOE_OK;
        }
        if (h > 0) {
            GemmParams dn{};
            dn.offsets = m->offsets; dn.order = m->order; dn.perm = m->perm; dn.E = E;
            dn.N = d; dn.K = h; dn.slots = T * K;
            dn.a = m->Aact; dn.lda = h; dn.c = m->O; dn.ldc = d;
            for (int e = 0; e < E; ++e) dn.w[e] = W_down[e];
            dn.ldb = h;
            dn.part = m->split; dn.resident = m->resident;
            dn.dpart = skinny ? m->dpart : nullptr;
            if (self) {
                dn.self_dispatch = 1;
                dn.idx = m->idx; dn.topk = K;
            }
            LAUNCH(TMT_MOE_PH_GEMM_DOWN, skinny ? launch_skinny_gemm(GEMM_DOWN, false, dn, T, s, &halves)
                                                : launch_gemm(GEMM_DOWN, false, dn, s));
        }
        CombineParams cp{};
        cp.O = h > 0 ? m->O : m->U; cp.slot_of = m->slot_of; cp.gate = m->gate;
        cp.Y = Y; cp.beta = beta; cp.T = T; cp.d = d; cp.K = K; cp.silu = h == 0;
        if (halves) {  // the decode GEMM_DOWN left two fp32 K halves; O is formed here
            cp.part = m->dpart; cp.O_out = m->O; cp.slots = T * K;
        }
        if (self) {
            cp.self_dispatch = 1; cp.idx = m->idx;
            DispatchTables& dt = cp.tables;
            dt.T = T; dt.E = E; dt.K = K; dt.probs = m->probs; dt.lse = m->lse;
            dt.offsets = m->offsets; dt.counts = m->counts; dt.order = m->order;
            dt.perm = m->perm; dt.slot_of = m->slot_of; dt.stats = m->stats;
        }
        LAUNCH(TMT_MOE_PH_COMBINE, launch_combine(cp, s));
    }
    m->last_T = T;
    return TMT_MOE_OK;
}

// Argument checks of the backward; `X` / `dX` name the block's input and its
// gradient (internal arena buffers for the LayerNorm variant).
int check_backward(tmt_moe* m, const uint16_t* dY, const uint16_t* X, const uint16_t* Wr,
                   const uint16_t* const* W_up, const uint16_t* const* W_down, const uint16_t* dX,
                   const float* dWr, float* const* dW_up, float* const* dW_down) {
    if (!m) return fail(TMT_MOE_EINVAL, "handle is NULL");
    const tmt_moe_desc& ds = m->desc;
    if (ds.weight_format != TMT_MOE_WEIGHTS_BF16)
        return fail(TMT_MOE_EINVAL, "backward needs bf16 weights");
    if (m->last_T < 0) return fail(TMT_MOE_ESTATE, "backward called without a successful forward");
    const int T = m->last_T, E = ds.experts, h = ds.hidden;
    if (T > 0 && (!dY || !X || !dX)) return fail(TMT_MOE_EINVAL, "dY, X and dX must be non-NULL");
    const unsigned a = m->align_bf16, af = m->align_f32;
    if (!aligned_to(dY, a) || !aligned_to(X, a) || !aligned_to(dX, a))
        return fail(TMT_MOE_EINVAL, "dY, X and dX must be %u-byte aligned", a);
    if (E > 1 && (!Wr || !dWr || !aligned_to(Wr, a) || !aligned_to(dWr, af)))
        return fail(TMT_MOE_EINVAL, "Wr and dWr must be aligned pointers (%u / %u bytes) when experts > 1", a, af);
    if (!aligned_to(dWr, af)) return fail(TMT_MOE_EINVAL, "dWr must be %u-byte aligned", af);
    int rc = check_ptrs((const void* const*)W_up, E, "W_up", a);
    if (rc) return rc;
    if ((rc = check_ptrs((const void* const*)dW_up, E, "dW_up", af))) return rc;
    if (h > 0) {
        if ((rc = check_ptrs((const void* const*)W_down, E, "W_down", a))) return rc;
        if ((rc = check_ptrs((const void* const*)dW_down, E, "dW_down", af))) return rc;
    }
    return check_device(m);
}

// Backward of the LayerNorm in front of the block (tmt_moe_backward_ln).
struct LnGrad {
    const uint16_t* S;
    const float* gamma;
    uint16_t* dS;
    float* dGamma;
    float* dBeta;
};

// The backward's launches (arguments checked). With `ln`, dX is the gradient
// at the LayerNorm output: for d <= kLnFusedMaxD the scatter consumes it in
// registers (dX is not written), otherwise it lands in dX and the two-pass
// LayerNorm backward follows.
int run_backward(tmt_moe* m, hipStream_t s, const uint16_t* dY, const uint16_t* X,
                 const uint16_t* Wr, const uint16_t* const* W_up, const uint16_t* const* W_down,
                 float aux_coef, float z_coef, uint16_t* dX, float* dWr, float* const* dW_up,
                 float* const* dW_down, const LnGrad* ln) {
    const tmt_moe_desc& ds = m->desc;
    const int T = m->last_T, E = ds.experts, K = ds.topk, d = ds.d, h = ds.hidden, hn = m->hn;

    if (T > 0) {
        CombineBwdParams cb{};
        cb.dY = dY; cb.O = h > 0 ? m->O : m->U; cb.slot_of = m->slot_of; cb.idx = m->idx;
        cb.gate = m->gate; cb.probs = m->probs; cb.lse = m->lse; cb.counts = m->counts;
        cb.T = T; cb.d = d; cb.E = E; cb.K = K; cb.silu = h == 0;
        cb.aux_coef = aux_coef; cb.z_coef = z_coef; cb.dO = m->dO; cb.dlogits = m->dlogits;
        cb.X = X; cb.Xg = m->Xg;
        LAUNCH(TMT_MOE_PH_COMBINE_BWD, launch_combine_bwd(cb, s));
    }
    if (h > 0) {
        if (T > 0) {
            GemmParams da{};
            da.offsets = m->offsets; da.order = m->order; da.perm = m->perm; da.E = E;
            da.N = h; da.K = d; da.slots = T * K;
            da.a = m->dO; da.lda = d; da.c = m->dU; da.ldc = h; da.u = m->U;
            for (int e = 0; e < E; ++e) da.w[e] = W_down[e];
            da.ldb = h;
            LAUNCH(TMT_MOE_PH_GEMM_DACT, launch_gemm(GEMM_DACT, false, da, s));
        }
        GemmParams dwd{};
        dwd.offsets = m->offsets; dwd.order = m->order; dwd.perm = m->perm; dwd.E = E;
        dwd.M = d; dwd.N = h;
        dwd.a = m->dO; dwd.lda = d; dwd.b = m->Aact; dwd.ldb = h; dwd.ldc = h;
        for (int e = 0; e < E; ++e) dwd.dw[e] = dW_down[e];
        LAUNCH(TMT_MOE_PH_GEMM_DW_DOWN, launch_gemm(GEMM_DW_DOWN, false, dwd, s));
    }
    GemmParams dwu{};
    dwu.offsets = m->offsets; dwu.order = m->order; dwu.perm = m->perm; dwu.E = E;
    dwu.M = hn; dwu.N = d;
    dwu.a = m->dU; dwu.lda = hn; dwu.b = m->Xg; dwu.ldb = d; dwu.ldc = d;
    for (int e = 0; e < E; ++e) dwu.dw[e] = dW_up[e];
    LAUNCH(TMT_MOE_PH_GEMM_DW_UP, launch_gemm(GEMM_DW_UP, false, dwu, s));
    if (T > 0) {
        GemmParams dx{};
        dx.offsets = m->offsets; dx.order = m->order; dx.perm = m->perm; dx.E = E;
        dx.N = d; dx.K = hn; dx.slots = T * K;
        dx.a = m->dU; dx.lda = hn; dx.c = m->dXg; dx.ldc = d;
        for (int e = 0; e < E; ++e) dx.w[e] = W_up[e];
        dx.ldb = d;
        dx.part = m->split; dx.resident = m->resident;
        if (m->wt != nullptr && gemm_tile(GEMM_DX, dx).m == 256) {
            // dXg = dU W_up as GEMM_DOWN over W_up^T: a transpose of the
            // weights (E * hn * d * 2 bytes each way) buys K-contiguous B
            // tiles for the GEMM (ds_read_b128 instead of the transposing
            // 8-byte reads, half the LDS read instructions)
            TransposeParams tp{};
            for (int e = 0; e < E; ++e) tp.src[e] = W_up[e];
            tp.ld_src = d; tp.rows = hn; tp.cols = d; tp.dst = m->wt;
            LAUNCH(TMT_MOE_PH_GEMM_DX, launch_transpose_bf16(tp, E, s));
            GemmParams dt = dx;
            for (int e = 0; e < E; ++e) dt.w[e] = m->wt + (int64_t)e * d * hn;
            dt.ldb = hn;
            LAUNCH(TMT_MOE_PH_GEMM_DX, launch_gemm(GEMM_DOWN, false, dt, s));
        } else {
            LAUNCH(TMT_MOE_PH_GEMM_DX, launch_gemm(GEMM_DX, false, dx, s));
        }
    }
    if (E == 1 && dWr) {
        // The dense path has no router; its gradient slot is zeroed like the
        // reference's (moe.cu:486-487).
        LAUNCH(TMT_MOE_PH_ROUTER_DW, launch_zero_f32(dWr, d, s));
    }
    // Without the LayerNorm the scatter's launch also runs the router weight
    // gradient's second pass (one launch fewer).
    RouterDwParams rw{};
    const bool dw_in_scatter = E > 1 && T > 0 && ln == nullptr;
    if (E > 1) {
        // With T == 0 the partial pass sums no rows and writes zeros.
        rw.dlogits = m->dlogits; rw.X = X; rw.T = T; rw.d = d; rw.E = E;
        rw.nchunks = router_dw_chunks(T, E, d); rw.partial = m->dwr_partial; rw.dWr = dWr;
        LAUNCH(TMT_MOE_PH_ROUTER_DW, launch_router_dw(rw, s, !dw_in_scatter));
    }
    // the scatter's fused LayerNorm backward needs the row width of the
    // LayerNorm itself (a padded handle runs the separate kernels)
    const bool ln_fused = ln != nullptr && d <= kLnFusedMaxD && !m->padded;
    if (T > 0) {
        ScatterParams sc{};
        sc.dXg = m->dXg; sc.slot_of = m->slot_of; sc.dlogits = E > 1 ? m->dlogits : nullptr;
        sc.Wr = Wr; sc.T = T; sc.d = d; sc.E = E; sc.K = K; sc.dX = dX;
        if (dw_in_scatter) sc.dw = rw;
        if (ln_fused) {
            sc.ln_S = ln->S; sc.ln_gamma = ln->gamma; sc.ln_mean = m->ln_mean; sc.ln_rstd = m->ln_rstd;
            sc.ln_dS = ln->dS; sc.ln_partial = m->ln_partial;
        }
        LAUNCH(TMT_MOE_PH_SCATTER, launch_scatter(sc, s));
    }
    if (ln_fused) {
        LAUNCH(TMT_MOE_PH_NORM_BWD, launch_colsum(m->ln_partial, T > 0 ? scatter_blocks(T) : 0, 2 * d,
                                                  m->ln_partial2, d, d, ln->dGamma, ln->dBeta, s));
    } else if (ln) {
        // the caller's S / dS rows have the caller's width; dX (the gradient
        // at H) has the internal one
        LayerNormParams lp{};
        lp.S = ln->S; lp.gamma = ln->gamma; lp.T = T; lp.d = m->user.d;
        lp.lds = m->user.d; lp.ldh = d;
        lp.mean = m->ln_mean; lp.rstd = m->ln_rstd; lp.dH = dX; lp.dS = ln->dS;
        lp.partial = m->ln_partial; lp.partial2 = m->ln_partial2; lp.dgamma = ln->dGamma; lp.dbeta = ln->dBeta;
        LAUNCH(TMT_MOE_PH_NORM_BWD, launch_ln_bwd(lp, s));
    }
    return TMT_MOE_OK;
}

int check_ln_shape(int32_t T, int32_t d) {
    if (T < 0) return fail(TMT_MOE_EINVAL, "T=%d must be >= 0", T);
    if (d < 1 || d > (1 << 20)) return fail(TMT_MOE_EINVAL, "d=%d must be in [1, 2^20]", d);
    return TMT_MOE_OK;
}

// Workspace of the standalone LayerNorm backward, in floats: chunk partials,
// then (from *level1_off, 256-byte aligned) the level-1 column sums.
size_t ln_workspace_floats(int32_t T, int32_t d, size_t* level1_off) {
    const size_t nch = (size_t)ln_chunks(T), pw = (size_t)ln_width4(d);
    const size_t off = (nch * 2 * pw + 63) & ~size_t(63);
    *level1_off = off;
    return off + (size_t)colsum_groups((int)nch) * 2 * pw;
}

int check_ln_backward_args(int32_t T, int32_t d, const uint16_t* S, const uint16_t* dH, const float* gamma,
                           const float* mean, const float* rstd, const uint16_t* dS, const float* dGamma,
                           const float* dBeta) {
    int rc = check_ln_shape(T, d);
    if (rc) return rc;
    if (T > 0 && (!S || !dH || !mean || !rstd || !dS))
        return fail(TMT_MOE_EINVAL, "S, dH, mean, rstd and dS must be non-NULL");
    if (!gamma || !dGamma || !dBeta) return fail(TMT_MOE_EINVAL, "gamma, dGamma and dBeta must be non-NULL");
    if (!aligned16(S) || !aligned16(dH) || !aligned16(dS) || !aligned16(gamma) || !aligned16(dGamma) ||
        !aligned16(dBeta))
        return fail(TMT_MOE_EINVAL, "S, dH, dS, gamma, dGamma and dBeta must be 16-byte aligned");
    return TMT_MOE_OK;
}

// The LayerNorm backward's launches over a workspace at `ws` (chunk
// partials, then the level-1 column sums from float offset `level1_off`).
// Every workspace element the kernels read is written by them first.
int run_ln_backward(hipStream_t s, int32_t T, int32_t d, const uint16_t* S, const uint16_t* dH,
                    const float* gamma, const float* mean, const float* rstd, uint16_t* dS, float* dGamma,
                    float* dBeta, float* ws, size_t level1_off) {
    LayerNormParams p{};
    p.S = S; p.gamma = gamma; p.T = T; p.d = d; p.lds = d; p.ldh = d; p.mean = const_cast<float*>(mean);
    p.rstd = const_cast<float*>(rstd); p.dH = dH; p.dS = dS;
    p.partial = ws;
    p.partial2 = ws + level1_off;
    p.dgamma = dGamma; p.dbeta = dBeta;
    HIP_TRY(launch_ln_bwd(p, s));
    return TMT_MOE_OK;
}

// ---- padded handles (d or hidden not a multiple of 64) ----------------------
// n matrices of rows_s x cols_s (contiguous rows) copied into rows_d x cols_d
// ones: zero-filled when the destination is larger, cropped when smaller.
int copy_mats(hipStream_t s, const void* const* src, void* const* dst, int n, int64_t rows_s, int64_t cols_s,
              int64_t rows_d, int64_t cols_d, int elem_bytes) {
    PadParams p{};
    for (int i = 0; i < n; ++i) {
        p.src[i] = src[i];
        p.dst[i] = dst[i];
    }
    p.rows_s = rows_s; p.cols_s = cols_s; p.ld_s = cols_s;
    p.rows_d = rows_d; p.cols_d = cols_d; p.ld_d = cols_d;
    HIP_TRY(launch_pad_copy(p, n, elem_bytes, s));
    return TMT_MOE_OK;
}
// [T][user d] bf16 rows to [T][d] and back.
int pad_rows(const tmt_moe* m, hipStream_t s, int T, const uint16_t* src, uint16_t* dst) {
    const void* a[1] = {src};
    void* b[1] = {dst};
    return copy_mats(s, a, b, 1, T, m->user.d, T, m->desc.d, 2);
}
int unpad_rows(const tmt_moe* m, hipStream_t s, int T, const uint16_t* src, uint16_t* dst) {
    const void* a[1] = {src};
    void* b[1] = {dst};
    return copy_mats(s, a, b, 1, T, m->desc.d, T, m->user.d, 2);
}
// Router and expert weights into the handle's padded copies.
int pad_weights(tmt_moe* m, hipStream_t s, const uint16_t* Wr, const uint16_t* const* W_up,
                const uint16_t* const* W_down) {
    const int E = m->desc.experts, du = m->user.d, dp = m->desc.d, hu = m->user.hidden, hp = m->desc.hidden;
    const int hnu = hu > 0 ? hu : du;
    int rc;
    if (E > 1) {
        const void* a[1] = {Wr};
        void* b[1] = {m->pwr};
        if ((rc = copy_mats(s, a, b, 1, E, du, E, dp, 2))) return rc;
    }
    if ((rc = copy_mats(s, (const void* const*)W_up, (void* const*)m->pwu, E, hnu, du, m->hn, dp, 2))) return rc;
    if (hp > 0 && (rc = copy_mats(s, (const void* const*)W_down, (void* const*)m->pwd, E, du, hu, dp, hp, 2)))
        return rc;
    return TMT_MOE_OK;
}
// Gradients from the padded copies to the caller's (dWr may be NULL when E == 1).
int unpad_grads(tmt_moe* m, hipStream_t s, float* dWr, float* const* dW_up, float* const* dW_down) {
    const int E = m->desc.experts, du = m->user.d, dp = m->desc.d, hu = m->user.hidden, hp = m->desc.hidden;
    const int hnu = hu > 0 ? hu : du;
    int rc;
    if (dWr) {
        const void* a[1] = {m->pdwr};
        void* b[1] = {dWr};
        if ((rc = copy_mats(s, a, b, 1, E, dp, E, du, 4))) return rc;
    }
    if ((rc = copy_mats(s, (const void* const*)m->pdwu, (void* const*)dW_up, E, m->hn, dp, hnu, du, 4))) return rc;
    if (hp > 0 && (rc = copy_mats(s, (const void* const*)m->pdwd, (void* const*)dW_down, E, dp, hp, du, hu, 4)))
        return rc;
    return TMT_MOE_OK;
}

}  // namespace

extern "C" {

const char* tmt_moe_last_error(void) { return g_last_error.c_str(); }

int tmt_moe_workspace_size(const tmt_moe_desc* desc, size_t* bytes) {
    int rc = validate_desc(desc);
    if (rc) return rc;
    if (!bytes) return fail(TMT_MOE_EINVAL, "bytes is NULL");
    const Sizes sz = plan(desc, nullptr);
    *bytes = sz.layer + sz.shared;
    return TMT_MOE_OK;
}

int tmt_moe_workspace_sizes(const tmt_moe_desc* desc, size_t* per_layer, size_t* shared) {
    int rc = validate_desc(desc);
    if (rc) return rc;
    const Sizes sz = plan(desc, nullptr);
    if (per_layer) *per_layer = sz.layer;
    if (shared) *shared = sz.shared;
    return TMT_MOE_OK;
}

namespace {
// Shared by tmt_moe_create (workspace == nullptr: the handle allocates its
// own) and tmt_moe_create_shared.
int create_handle(const tmt_moe_desc* desc, void* workspace, size_t workspace_bytes, tmt_moe** out) {
    if (!out) return fail(TMT_MOE_EINVAL, "out is NULL");
    *out = nullptr;
    int rc = validate_desc(desc);
    if (rc) return rc;
    const Sizes sz = plan(desc, nullptr);
    if (workspace) {
        if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
            return fail(TMT_MOE_EINVAL, "the shared workspace must be 256-byte aligned");
        if (workspace_bytes < sz.shared)
            return fail(TMT_MOE_EINVAL, "shared workspace of %zu bytes is smaller than the %zu bytes this layer needs",
                        workspace_bytes, sz.shared);
    }
    tmt_moe* m = new (std::nothrow) tmt_moe();
    if (!m) return fail(TMT_MOE_ENOMEM, "host allocation failed");
    m->desc = internal_desc(*desc);
    m->user = *desc;
    m->hn = m->desc.hidden > 0 ? m->desc.hidden : m->desc.d;
    if (is_padded(*desc)) {
        // operands are read element by element into the padded copies
        m->align_bf16 = 2;
        m->align_f32 = 4;
    }
    hipError_t err = hipGetDevice(&m->device);
    if (err != hipSuccess) {
        delete m;
        return fail(TMT_MOE_EDEVICE, "hipGetDevice failed: %s", hipGetErrorString(err));
    }
    m->own_ws = workspace == nullptr;
    m->arena_bytes = sz.layer + (m->own_ws ? sz.shared : 0);
    err = hipMalloc(&m->arena, m->arena_bytes);
    if (err != hipSuccess) {
        delete m;
        (void)hipGetLastError();
        return fail(TMT_MOE_ENOMEM, "hipMalloc(%zu) failed: %s", m->arena_bytes, hipGetErrorString(err));
    }
    m->ws = m->own_ws ? m->arena + sz.layer : static_cast<char*>(workspace);
    plan(desc, m);
    // The decode router's ticket starts at zero (each call leaves it at zero).
    err = hipMemset(m->ticket, 0, sizeof(int32_t));
    if (err == hipSuccess) err = hipStreamSynchronize(nullptr);
    if (err != hipSuccess) {
        (void)hipFree(m->arena);
        delete m;
        (void)hipGetLastError();
        return fail(TMT_MOE_EDEVICE, "initialising the workspace failed: %s", hipGetErrorString(err));
    }
    *out = m;
    return TMT_MOE_OK;
}
}  // namespace

int tmt_moe_create(const tmt_moe_desc* desc, tmt_moe** out) {
    return create_handle(desc, nullptr, 0, out);
}

int tmt_moe_create_shared(const tmt_moe_desc* desc, void* workspace, size_t workspace_bytes, tmt_moe** out) {
    if (!workspace) {
        if (out) *out = nullptr;
        return fail(TMT_MOE_EINVAL, "workspace is NULL (use tmt_moe_create for a private one)");
    }
    return create_handle(desc, workspace, workspace_bytes, out);
}

int tmt_moe_destroy(tmt_moe* m) {
    if (!m) return TMT_MOE_OK;
    hipError_t err = hipSuccess;
    for (hipEvent_t ev : m->prof_events) (void)hipEventDestroy(ev);
    if (m->arena) err = hipFree(m->arena);
    delete m;
    if (err != hipSuccess) return fail(TMT_MOE_EDEVICE, "hipFree failed: %s", hipGetErrorString(err));
    return TMT_MOE_OK;
}

int tmt_moe_forward(tmt_moe* m, void* stream, int32_t T, const uint16_t* X,
                    const uint16_t* Wr, const float* logit_bias,
                    const uint16_t* const* W_up, const uint16_t* const* W_down,
                    uint16_t* Y, float beta) {
    int rc = check_forward(m, T, X, "X", Wr, W_up, W_down, Y);
    if (rc) return rc;
    m->last_ln = false;
    hipStream_t s = (hipStream_t)stream;
    if (!m->padded) return run_forward(m, s, T, X, Wr, logit_bias, W_up, W_down, Y, beta);
    m->last_T = -1;
    if ((rc = pad_weights(m, s, Wr, W_up, W_down)) || (rc = pad_rows(m, s, T, X, m->px))) return rc;
    if (beta != 0.0f && (rc = pad_rows(m, s, T, Y, m->py))) return rc;  // beta == 0: Y is not read
    if ((rc = run_forward(m, s, T, m->px, m->pwr, logit_bias, m->pwu, m->pwd, m->py, beta))) return rc;
    return unpad_rows(m, s, T, m->py, Y);
}

int tmt_moe_forward_ln(tmt_moe* m, void* stream, int32_t T, const uint16_t* S,
                       const float* ln_gamma, const float* ln_beta,
                       const uint16_t* Wr, const float* logit_bias,
                       const uint16_t* const* W_up, const uint16_t* const* W_down,
                       uint16_t* Y, float beta) {
    int rc = check_forward(m, T, S, "S", Wr, W_up, W_down, Y);
    if (rc) return rc;
    if (!ln_gamma || !ln_beta || !aligned16(ln_gamma) || !aligned16(ln_beta))
        return fail(TMT_MOE_EINVAL, "ln_gamma and ln_beta must be 16-byte aligned device pointers");
    hipStream_t s = (hipStream_t)stream;
    m->last_T = -1;
    m->last_ln = false;
    // H has the internal width (zeros in the padded columns of a padded handle)
    LayerNormParams ln{};
    ln.S = S; ln.gamma = ln_gamma; ln.beta = ln_beta; ln.T = T; ln.d = m->user.d;
    ln.lds = m->user.d; ln.ldh = m->desc.d;
    ln.H = m->H; ln.mean = m->ln_mean; ln.rstd = m->ln_rstd;
    // Routed batches: the router normalises its rows itself (one read of S
    // instead of a LayerNorm pass and a read of H); otherwise the LayerNorm
    // runs first. Batches whose logits come from the matrix cores also take
    // the separate pass: at c3 the LayerNorm pass plus the matrix-core router
    // over H is faster than the VALU router normalising S itself.
    const LnFuse fuse{S, ln_gamma, ln_beta};
    const bool fused = !m->padded && ln_in_router(T, m->desc.experts, m->desc.d) &&
                       !router_mfma_fits(T, m->desc.experts, m->desc.topk, m->desc.d);
    if (!fused) LAUNCH(TMT_MOE_PH_NORM, launch_ln_fwd(ln, s));
    if (m->padded) {
        if ((rc = pad_weights(m, s, Wr, W_up, W_down))) return rc;
        if (beta != 0.0f && (rc = pad_rows(m, s, T, Y, m->py))) return rc;
        if ((rc = run_forward(m, s, T, m->H, m->pwr, logit_bias, m->pwu, m->pwd, m->py, beta))) return rc;
        if ((rc = unpad_rows(m, s, T, m->py, Y))) return rc;
    } else if ((rc = run_forward(m, s, T, m->H, Wr, logit_bias, W_up, W_down, Y, beta, fused ? &fuse : nullptr))) {
        return rc;
    }
    m->last_ln = true;
    return TMT_MOE_OK;
}

int tmt_moe_forward_mxfp4(tmt_moe* m, void* stream, int32_t T, const uint16_t* X,
                          const uint16_t* Wr, const float* logit_bias,
                          const uint8_t* const* W_up, const uint8_t* const* W_up_scale,
                          const uint8_t* const* W_down, const uint8_t* const* W_down_scale,
                          uint16_t* Y, float beta) {
    if (!m) return fail(TMT_MOE_EINVAL, "handle is NULL");
    const tmt_moe_desc& ds = m->desc;
    if (ds.weight_format != TMT_MOE_WEIGHTS_MXFP4 && !is_mx(ds.weight_format))
        return fail(TMT_MOE_EINVAL, "handle expects bf16 weights: use tmt_moe_forward");
    if (T < 0 || T > ds.max_tokens) return fail(TMT_MOE_EINVAL, "T=%d outside [0, %d]", T, ds.max_tokens);
    const int E = ds.experts, K = ds.topk, d = ds.d, h = ds.hidden;
    if (T > 0 && (!X || !Y)) return fail(TMT_MOE_EINVAL, "X and Y must be non-NULL");
    if (!aligned16(X) || !aligned16(Y)) return fail(TMT_MOE_EINVAL, "X and Y must be 16-byte aligned");
    if (E > 1 && (!Wr || !aligned16(Wr))) return fail(TMT_MOE_EINVAL, "Wr must be a 16-byte aligned pointer when experts > 1");
    int rc;
    if ((rc = check_ptrs((const void* const*)W_up, E, "W_up"))) return rc;
    if ((rc = check_ptrs((const void* const*)W_up_scale, E, "W_up_scale"))) return rc;
    if ((rc = check_ptrs((const void* const*)W_down, E, "W_down"))) return rc;
    if ((rc = check_ptrs((const void* const*)W_down_scale, E, "W_down_scale"))) return rc;
    if ((rc = check_device(m))) return rc;
    hipStream_t s = (hipStream_t)stream;
    m->last_T = -1;
    m->last_ln = false;
    if ((rc = route(m, s, T, X, Wr, logit_bias))) return rc;
    if (T > 0 && is_mx(ds.weight_format)) {
        const int TK = T * K;
        const int64_t srows = (int64_t)ds.max_tokens * K + kMxScalePadRows;
        // X is rounded once per token and written to the token's K slots, so
        // that every up-GEMM tile reads one contiguous block per K step.
        MxQuantParams qp{};
        qp.X = X; qp.ldx = d; qp.rows = T; qp.K = d;
        qp.slot_of = E > 1 ? m->slot_of : nullptr; qp.copies = E > 1 ? K : 1;
        qp.codes = m->xq; qp.scales = m->xq_scales; qp.srows = srows;
        LAUNCH(TMT_MOE_PH_GEMM_UP, launch_mx_quant_rows(qp, s));
        // the weight codes of both GEMMs in K planes, so that a tile's K step
        // is one contiguous block: given so (MX_PLANES), or copied here (one
        // launch, counted in the up phase)
        const uint8_t* wup_pl[kMaxExperts];
        const uint8_t* wdn_pl[kMaxExperts];
        if (ds.weight_format == TMT_MOE_WEIGHTS_MXFP4_MX_PLANES) {
            for (int e = 0; e < E; ++e) { wup_pl[e] = W_up[e]; wdn_pl[e] = W_down[e]; }
        } else {
            MxPlanesParams wp{};
            for (int e = 0; e < E; ++e) { wp.src[0][e] = W_up[e]; wp.src[1][e] = W_down[e]; }
            wp.dst[0] = m->wplanes;
            wp.dst[1] = m->wplanes + (size_t)E * h * d / 2;
            wp.N[0] = h; wp.K[0] = d; wp.N[1] = d; wp.K[1] = h; wp.E = E;
            LAUNCH(TMT_MOE_PH_GEMM_UP, launch_mx_weight_planes(wp, s));
            for (int e = 0; e < E; ++e) {
                wup_pl[e] = wp.dst[0] + (size_t)e * h * d / 2;
                wdn_pl[e] = wp.dst[1] + (size_t)e * d * h / 2;
            }
        }
        MxGemmParams up{};
        up.offsets = m->offsets; up.E = E; up.N = h; up.K = d; up.slots = TK;
        up.a_codes = m->xq; up.a_scales = m->xq_scales; up.a_srows = srows;
        for (int e = 0; e < E; ++e) { up.wq[e] = wup_pl[e]; up.wsc[e] = W_up_scale[e]; }
        up.q_codes = m->aq; up.q_scales = m->aq_scales; up.q_srows = srows;
        LAUNCH(TMT_MOE_PH_GEMM_UP, launch_mx_gemm(true, up, s));
        MxGemmParams dn{};
        dn.offsets = m->offsets; dn.E = E; dn.N = d; dn.K = h; dn.slots = TK;
        dn.a_codes = m->aq; dn.a_scales = m->aq_scales; dn.a_srows = srows;
        for (int e = 0; e < E; ++e) { dn.wq[e] = wdn_pl[e]; dn.wsc[e] = W_down_scale[e]; }
        dn.c = m->O; dn.ldc = d;
        LAUNCH(TMT_MOE_PH_GEMM_DOWN, launch_mx_gemm(false, dn, s));
        CombineParams cp{};
        cp.O = m->O; cp.slot_of = m->slot_of; cp.gate = m->gate;
        cp.Y = Y; cp.beta = beta; cp.T = T; cp.d = d; cp.K = K; cp.silu = 0;
        LAUNCH(TMT_MOE_PH_COMBINE, launch_combine(cp, s));
    } else if (T > 0) {
        GemmParams up{};
        up.offsets = m->offsets; up.order = m->order; up.perm = m->perm; up.E = E;
        up.N = h; up.K = d; up.slots = T * K;
        up.a = X; up.lda = d; up.c = nullptr; up.ldc = h; up.c2 = m->Aact;  // no backward: silu'(U) not kept
        for (int e = 0; e < E; ++e) { up.wq[e] = W_up[e]; up.wsc[e] = W_up_scale[e]; }
        LAUNCH(TMT_MOE_PH_GEMM_UP, launch_gemm(GEMM_UP_FP4, true, up, s));
        GemmParams dn{};
        dn.offsets = m->offsets; dn.order = m->order; dn.perm = m->perm; dn.E = E;
        dn.N = d; dn.K = h; dn.slots = T * K;
        dn.a = m->Aact; dn.lda = h; dn.c = m->O; dn.ldc = d;
        for (int e = 0; e < E; ++e) { dn.wq[e] = W_down[e]; dn.wsc[e] = W_down_scale[e]; }
        LAUNCH(TMT_MOE_PH_GEMM_DOWN, launch_gemm(GEMM_DOWN_FP4, false, dn, s));
        CombineParams cp{};
        cp.O = m->O; cp.slot_of = m->slot_of; cp.gate = m->gate;
        cp.Y = Y; cp.beta = beta; cp.T = T; cp.d = d; cp.K = K; cp.silu = 0;
        LAUNCH(TMT_MOE_PH_COMBINE, launch_combine(cp, s));
    }
    m->last_T = T;
    return TMT_MOE_OK;
}

int tmt_moe_backward(tmt_moe* m, void* stream, const uint16_t* dY, const uint16_t* X,
                     const uint16_t* Wr, const uint16_t* const* W_up,
                     const uint16_t* const* W_down, float aux_coef, float z_coef,
                     uint16_t* dX, float* dWr, float* const* dW_up, float* const* dW_down) {
    // After tmt_moe_forward_ln the router ran on the internal LayerNorm output,
    // which the caller cannot pass as X: that forward pairs with
    // tmt_moe_backward_ln only.
    if (m && m->last_T >= 0 && m->last_ln)
        return fail(TMT_MOE_ESTATE, "the last forward was tmt_moe_forward_ln: use tmt_moe_backward_ln");
    int rc = check_backward(m, dY, X, Wr, W_up, W_down, dX, dWr, dW_up, dW_down);
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    if (!m->padded)
        return run_backward(m, s, dY, X, Wr, W_up, W_down, aux_coef, z_coef, dX, dWr, dW_up, dW_down, nullptr);
    const int T = m->last_T;
    if ((rc = pad_weights(m, s, Wr, W_up, W_down)) || (rc = pad_rows(m, s, T, X, m->px)) ||
        (rc = pad_rows(m, s, T, dY, m->pdy)))
        return rc;
    if ((rc = run_backward(m, s, m->pdy, m->px, m->pwr, m->pwu, m->pwd, aux_coef, z_coef, m->pdx,
                           dWr ? m->pdwr : nullptr, m->pdwu, m->pdwd, nullptr)))
        return rc;
    if ((rc = unpad_rows(m, s, T, m->pdx, dX))) return rc;
    return unpad_grads(m, s, dWr, dW_up, dW_down);
}

int tmt_moe_backward_ln(tmt_moe* m, void* stream, const uint16_t* dY, const uint16_t* S,
                        const float* ln_gamma, const uint16_t* Wr, const uint16_t* const* W_up,
                        const uint16_t* const* W_down, float aux_coef, float z_coef,
                        uint16_t* dS, float* dGamma, float* dBeta, float* dWr,
                        float* const* dW_up, float* const* dW_down) {
    if (!m) return fail(TMT_MOE_EINVAL, "handle is NULL");
    if (m->last_T >= 0 && !m->last_ln)
        return fail(TMT_MOE_ESTATE, "tmt_moe_backward_ln must follow tmt_moe_forward_ln");
    int rc = check_backward(m, dY, m->H, Wr, W_up, W_down, m->dH, dWr, dW_up, dW_down);
    if (rc) return rc;
    const int T = m->last_T;
    if (T > 0 && (!S || !dS)) return fail(TMT_MOE_EINVAL, "S and dS must be non-NULL");
    if (!aligned_to(S, m->align_bf16) || !aligned_to(dS, m->align_bf16))
        return fail(TMT_MOE_EINVAL, "S and dS must be %u-byte aligned", m->align_bf16);
    if (!ln_gamma || !dGamma || !dBeta || !aligned16(ln_gamma) || !aligned16(dGamma) || !aligned16(dBeta))
        return fail(TMT_MOE_EINVAL, "ln_gamma, dGamma and dBeta must be 16-byte aligned device pointers");
    const LnGrad lg{S, ln_gamma, dS, dGamma, dBeta};
    hipStream_t s = (hipStream_t)stream;
    if (!m->padded)
        return run_backward(m, s, dY, m->H, Wr, W_up, W_down, aux_coef, z_coef, m->dH, dWr, dW_up, dW_down, &lg);
    if ((rc = pad_weights(m, s, Wr, W_up, W_down)) || (rc = pad_rows(m, s, T, dY, m->pdy))) return rc;
    if ((rc = run_backward(m, s, m->pdy, m->H, m->pwr, m->pwu, m->pwd, aux_coef, z_coef, m->dH,
                           dWr ? m->pdwr : nullptr, m->pdwu, m->pdwd, &lg)))
        return rc;
    return unpad_grads(m, s, dWr, dW_up, dW_down);
}

int tmt_moe_read_stats(tmt_moe* m, void* stream, float* aux, float* z, int32_t* counts) {
    if (!m) return fail(TMT_MOE_EINVAL, "handle is NULL");
    if (m->last_T < 0) return fail(TMT_MOE_ESTATE, "no forward has run on this handle");
    int rc = check_device(m);
    if (rc) return rc;
    HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    const int E = m->desc.experts;
    float st[2 + kMaxExperts];
    HIP_TRY(hipMemcpy(st, m->stats, (size_t)(2 + E) * 4, hipMemcpyDeviceToHost));
    if (aux) *aux = st[0];
    if (z) *z = st[1];
    if (counts) std::memcpy(counts, st + 2, (size_t)E * 4);
    return TMT_MOE_OK;
}

int tmt_moe_set_profiling(tmt_moe* m, int enable) {
    if (!m) return fail(TMT_MOE_EINVAL, "handle is NULL");
    if (enable && m->prof_events.empty()) {
        m->prof_events.resize(2 * kProfPairs);
        for (auto& ev : m->prof_events) HIP_TRY(hipEventCreate(&ev));
    }
    if (!enable && m->prof_on) {
        int rc = prof_flush(m);
        if (rc) return rc;
    }
    m->prof_on = enable != 0;
    return TMT_MOE_OK;
}

int tmt_moe_read_profile(tmt_moe* m, float* ms, int32_t* launches, int reset) {
    if (!m) return fail(TMT_MOE_EINVAL, "handle is NULL");
    int rc = prof_flush(m);
    if (rc) return rc;
    for (int i = 0; i < TMT_MOE_NPHASES; ++i) {
        if (ms) ms[i] = (float)m->prof_ms[i];
        if (launches) launches[i] = m->prof_cnt[i];
        if (reset) {
            m->prof_ms[i] = 0.0;
            m->prof_cnt[i] = 0;
        }
    }
    return TMT_MOE_OK;
}

const char* tmt_moe_phase_name(int phase) {
    static const char* names[TMT_MOE_NPHASES] = {
        "router", "scan", "permute", "gemm_up", "gemm_down", "combine", "combine_bwd",
        "gemm_dact", "gemm_dw_down", "gemm_dw_up", "gemm_dx", "router_dw", "scatter",
        "norm", "norm_bwd"};
    return (phase >= 0 && phase < TMT_MOE_NPHASES) ? names[phase] : "unknown";
}

int tmt_moe_stats_device_ptr(tmt_moe* m, const void** ptr) {
    if (!m || !ptr) return fail(TMT_MOE_EINVAL, "handle or ptr is NULL");
    *ptr = m->stats;
    return TMT_MOE_OK;
}

int tmt_moe_read_routing(tmt_moe* m, void* stream, float* logits, float* probs,
                         int32_t* idx, float* gate, int32_t* offsets, int32_t* perm,
                         int32_t* slot_of) {
    if (!m) return fail(TMT_MOE_EINVAL, "handle is NULL");
    if (m->last_T < 0) return fail(TMT_MOE_ESTATE, "no forward has run on this handle");
    int rc = check_device(m);
    if (rc) return rc;
    HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    const int64_t T = m->last_T, E = m->desc.experts, K = m->desc.topk;
    if (E > 1) {
        if (logits && T) HIP_TRY(hipMemcpy(logits, m->logits, T * E * 4, hipMemcpyDeviceToHost));
        if (probs && T) HIP_TRY(hipMemcpy(probs, m->probs, T * E * 4, hipMemcpyDeviceToHost));
        if (idx && T) HIP_TRY(hipMemcpy(idx, m->idx, T * K * 4, hipMemcpyDeviceToHost));
    } else {
        if (logits) std::memset(logits, 0, T * E * 4);
        if (probs) for (int64_t i = 0; i < T; ++i) probs[i] = 1.0f;
        if (idx) std::memset(idx, 0, T * K * 4);
    }
    if (gate && T) HIP_TRY(hipMemcpy(gate, m->gate, T * K * 4, hipMemcpyDeviceToHost));
    if (offsets) HIP_TRY(hipMemcpy(offsets, m->offsets, (E + 1) * 4, hipMemcpyDeviceToHost));
    if (perm && T) HIP_TRY(hipMemcpy(perm, m->perm, T * K * 4, hipMemcpyDeviceToHost));
    if (slot_of && T) HIP_TRY(hipMemcpy(slot_of, m->slot_of, T * K * 4, hipMemcpyDeviceToHost));
    return TMT_MOE_OK;
}

int tmt_moe_layernorm_workspace_size(int32_t T, int32_t d, size_t* bytes) {
    int rc = check_ln_shape(T, d);
    if (rc) return rc;
    if (!bytes) return fail(TMT_MOE_EINVAL, "bytes is NULL");
    size_t off;
    *bytes = ln_workspace_floats(T, d, &off) * 4;
    return TMT_MOE_OK;
}

int tmt_moe_layernorm_forward(void* stream, int32_t T, int32_t d, const uint16_t* S, const float* gamma,
                              const float* beta, uint16_t* H, float* mean, float* rstd) {
    int rc = check_ln_shape(T, d);
    if (rc) return rc;
    if (T > 0 && (!S || !H || !mean || !rstd)) return fail(TMT_MOE_EINVAL, "S, H, mean and rstd must be non-NULL");
    if (!gamma || !beta) return fail(TMT_MOE_EINVAL, "gamma and beta must be non-NULL");
    if (!aligned16(S) || !aligned16(H) || !aligned16(gamma) || !aligned16(beta))
        return fail(TMT_MOE_EINVAL, "S, H, gamma and beta must be 16-byte aligned");
    LayerNormParams p{};
    p.S = S; p.gamma = gamma; p.beta = beta; p.T = T; p.d = d; p.lds = d; p.ldh = d;
    p.H = H; p.mean = mean; p.rstd = rstd;
    HIP_TRY(launch_ln_fwd(p, (hipStream_t)stream));
    return TMT_MOE_OK;
}

int tmt_moe_layernorm_backward(void* stream, int32_t T, int32_t d, const uint16_t* S, const uint16_t* dH,
                               const float* gamma, const float* mean, const float* rstd, uint16_t* dS,
                               float* dGamma, float* dBeta, void* workspace, size_t workspace_bytes) {
    int rc = check_ln_backward_args(T, d, S, dH, gamma, mean, rstd, dS, dGamma, dBeta);
    if (rc) return rc;
    size_t off;
    const size_t need = ln_workspace_floats(T, d, &off) * 4;
    if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
        return fail(TMT_MOE_EINVAL, "workspace must be a 256-byte aligned device pointer");
    if (workspace_bytes < need)
        return fail(TMT_MOE_EINVAL, "workspace of %zu bytes is smaller than the %zu bytes needed", workspace_bytes, need);
    return run_ln_backward((hipStream_t)stream, T, d, S, dH, gamma, mean, rstd, dS, dGamma, dBeta,
                           static_cast<float*>(workspace), off);
}

int tmt_moe_layernorm_backward_noalloc(void* stream, int32_t T, int32_t d, const uint16_t* S,
                                       const uint16_t* dH, const float* gamma, const float* mean,
                                       const float* rstd, uint16_t* dS, float* dGamma, float* dBeta) {
    int rc = check_ln_backward_args(T, d, S, dH, gamma, mean, rstd, dS, dGamma, dBeta);
    if (rc) return rc;
    size_t off;
    const size_t need = ln_workspace_floats(T, d, &off) * 4;
    if (need > kNoAllocScratchBytes)
        return fail(TMT_MOE_EINVAL,
                    "T=%d, d=%d needs %zu bytes of scratch, more than the %zu bytes this entry point holds",
                    T, d, need, kNoAllocScratchBytes);
    float* ws = nullptr;
    if ((rc = scratch_on_current_device(&ws))) return rc;
    return run_ln_backward((hipStream_t)stream, T, d, S, dH, gamma, mean, rstd, dS, dGamma, dBeta, ws, off);
}

int tmt_moe_f32_to_bf16(void* stream, const float* in, uint16_t* out, int64_t n) {
    if (n < 0) return fail(TMT_MOE_EINVAL, "n=%lld < 0", (long long)n);
    if (n > 0 && (!in || !out)) return fail(TMT_MOE_EINVAL, "in and out must be non-NULL");
    HIP_TRY(launch_f32_to_bf16(in, out, n, (hipStream_t)stream));
    return TMT_MOE_OK;
}

int tmt_moe_mxfp4_planes(void* stream, const uint8_t* codes, int32_t N, int32_t K, uint8_t* planes) {
    if (N <= 0 || K <= 0 || N % 64 != 0 || K % 64 != 0)
        return fail(TMT_MOE_EINVAL, "N=%d and K=%d must be positive multiples of 64", N, K);
    if ((int64_t)N * (K / 2) >= (int64_t(1) << 31)) return fail(TMT_MOE_EINVAL, "N*K/2 must fit in int32");
    if (!codes || !planes) return fail(TMT_MOE_EINVAL, "codes and planes must be non-NULL");
    if (!aligned16(codes) || !aligned16(planes)) return fail(TMT_MOE_EINVAL, "codes and planes must be 16-byte aligned");
    if (codes == planes) return fail(TMT_MOE_EINVAL, "codes and planes must not be the same buffer");
    MxPlanesParams p{};
    p.src[0][0] = codes;
    p.dst[0] = planes;
    p.N[0] = N;
    p.K[0] = K;
    p.E = 1;  // set 1 empty (N = 0)
    HIP_TRY(launch_mx_weight_planes(p, (hipStream_t)stream));
    return TMT_MOE_OK;
}

int tmt_moe_read_norm(tmt_moe* m, void* stream, uint16_t* H, float* mean, float* rstd) {
    if (!m) return fail(TMT_MOE_EINVAL, "handle is NULL");
    if (m->last_T < 0 || !m->last_ln) return fail(TMT_MOE_ESTATE, "the last forward was not tmt_moe_forward_ln");
    int rc = check_device(m);
    if (rc) return rc;
    HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    const int64_t T = m->last_T, du = m->user.d, dp = m->desc.d;
    if (H && T) HIP_TRY(hipMemcpy2D(H, du * 2, m->H, dp * 2, du * 2, T, hipMemcpyDeviceToHost));
    if (mean && T) HIP_TRY(hipMemcpy(mean, m->ln_mean, T * 4, hipMemcpyDeviceToHost));
    if (rstd && T) HIP_TRY(hipMemcpy(rstd, m->ln_rstd, T * 4, hipMemcpyDeviceToHost));
    return TMT_MOE_OK;
}

}  // extern "C"

// ------------------------------------------------------------------ AdamW --

struct tmt_moe_adamw {
    int device = 0;
    char* arena = nullptr;  // chunk table, per-chunk sums, sumsq
    AdamwParams p{};
};

namespace {
int adamw_check_device(const tmt_moe_adamw* o) {
    int dev = -1;
    HIP_TRY(hipGetDevice(&dev));
    if (dev != o->device)
        return fail(TMT_MOE_EINVAL, "optimizer was created on device %d but device %d is current", o->device, dev);
    return TMT_MOE_OK;
}
}  // namespace

extern "C" {

int tmt_moe_adamw_create(const tmt_moe_adamw_param* params, int32_t count, tmt_moe_adamw** out) {
    if (!out) return fail(TMT_MOE_EINVAL, "out is NULL");
    *out = nullptr;
    if (count < 0 || (count > 0 && !params)) return fail(TMT_MOE_EINVAL, "bad parameter list (count=%d)", count);
    std::vector<AdamwChunk> chunks;
    for (int i = 0; i < count; ++i) {
        const tmt_moe_adamw_param& q = params[i];
        if (q.n < 0) return fail(TMT_MOE_EINVAL, "parameter %d: n=%lld < 0", i, (long long)q.n);
        if (q.flags < 0 || q.flags > 3) return fail(TMT_MOE_EINVAL, "parameter %d: unknown flags %d", i, q.flags);
        if (q.n > 0 && (!q.master || !q.m || !q.v || !q.grad))
            return fail(TMT_MOE_EINVAL, "parameter %d: master, m, v and grad must be non-NULL", i);
        if (!aligned16(q.master) || !aligned16(q.m) || !aligned16(q.v) || !aligned16(q.grad) || !aligned16(q.work))
            return fail(TMT_MOE_EINVAL, "parameter %d: pointers must be 16-byte aligned", i);
        for (int64_t s = 0; s < q.n; s += kAdamChunk) {
            AdamwChunk c{};
            c.master = q.master + s; c.m = q.m + s; c.v = q.v + s; c.grad = q.grad + s;
            c.work = q.work ? q.work + s : nullptr;
            c.len = (int32_t)std::min<int64_t>(kAdamChunk, q.n - s);
            c.flags = q.flags;
            chunks.push_back(c);
        }
    }
    if (chunks.size() > (size_t)INT32_MAX) return fail(TMT_MOE_EINVAL, "too many chunks");
    tmt_moe_adamw* o = new (std::nothrow) tmt_moe_adamw();
    if (!o) return fail(TMT_MOE_ENOMEM, "host allocation failed");
    hipError_t err = hipGetDevice(&o->device);
    const size_t nch = chunks.size();
    Layout L;
    const size_t o_tab = L.add(nch * sizeof(AdamwChunk)), o_part = L.add(nch * 8), o_sum = L.add(8);
    if (err == hipSuccess) err = hipMalloc(&o->arena, L.total);
    if (err != hipSuccess) {
        delete o;
        (void)hipGetLastError();
        return fail(TMT_MOE_ENOMEM, "optimizer allocation failed: %s", hipGetErrorString(err));
    }
    o->p.chunks = reinterpret_cast<AdamwChunk*>(o->arena + o_tab);
    o->p.nchunks = (int)nch;
    o->p.partial = reinterpret_cast<double*>(o->arena + o_part);
    o->p.sumsq = reinterpret_cast<double*>(o->arena + o_sum);
    if (nch) err = hipMemcpy(o->arena + o_tab, chunks.data(), nch * sizeof(AdamwChunk), hipMemcpyHostToDevice);
    if (err == hipSuccess) err = hipMemset(o->arena + o_sum, 0, sizeof(double));
    if (err == hipSuccess) err = hipStreamSynchronize(nullptr);
    if (err != hipSuccess) {
        (void)hipFree(o->arena);
        delete o;
        (void)hipGetLastError();
        return fail(TMT_MOE_EDEVICE, "initialising the optimizer failed: %s", hipGetErrorString(err));
    }
    *out = o;
    return TMT_MOE_OK;
}

int tmt_moe_adamw_destroy(tmt_moe_adamw* o) {
    if (!o) return TMT_MOE_OK;
    hipError_t err = o->arena ? hipFree(o->arena) : hipSuccess;
    delete o;
    if (err != hipSuccess) return fail(TMT_MOE_EDEVICE, "hipFree failed: %s", hipGetErrorString(err));
    return TMT_MOE_OK;
}

int tmt_moe_adamw_step(tmt_moe_adamw* o, void* stream, float clip, float lr, float beta1, float beta2,
                       float eps, float weight_decay, int32_t step) {
    if (!o) return fail(TMT_MOE_EINVAL, "optimizer is NULL");
    if (step < 1) return fail(TMT_MOE_EINVAL, "step=%d must be >= 1 (1-based update count)", step);
    int rc = adamw_check_device(o);
    if (rc) return rc;
    AdamwHyper h{};
    h.clip = clip; h.lr = lr; h.b1 = beta1; h.b2 = beta2; h.eps = eps; h.wd = weight_decay;
    h.bc1 = 1.0f - powf(beta1, (float)step);
    h.bc2 = 1.0f - powf(beta2, (float)step);
    hipStream_t s = (hipStream_t)stream;
    HIP_TRY(launch_adamw_sumsq(o->p, s));
    HIP_TRY(launch_adamw_update(o->p, h, s));
    return TMT_MOE_OK;
}

int tmt_moe_adamw_read_sumsq(tmt_moe_adamw* o, void* stream, double* sumsq) {
    if (!o || !sumsq) return fail(TMT_MOE_EINVAL, "optimizer or sumsq is NULL");
    int rc = adamw_check_device(o);
    if (rc) return rc;
    HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    HIP_TRY(hipMemcpy(sumsq, o->p.sumsq, 8, hipMemcpyDeviceToHost));
    return TMT_MOE_OK;
}

int tmt_moe_adamw_zero_grads(tmt_moe_adamw* o, void* stream) {
    if (!o) return fail(TMT_MOE_EINVAL, "optimizer is NULL");
    int rc = adamw_check_device(o);
    if (rc) return rc;
    HIP_TRY(launch_adamw_zero(o->p, (hipStream_t)stream));
    return TMT_MOE_OK;
}

int tmt_moe_adamw_chunks(tmt_moe_adamw* o, int32_t* chunks) {
    if (!o || !chunks) return fail(TMT_MOE_EINVAL, "optimizer or chunks is NULL");
    *chunks = o->p.nchunks;
    return TMT_MOE_OK;
}

}  // extern "C"
