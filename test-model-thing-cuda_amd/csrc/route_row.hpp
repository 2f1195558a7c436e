// route_row.hpp -- routing of single token rows, shared by the decode
// router (router.hip) and the one-token up GEMM that routes its token itself
// (skinny.hip).
#pragma once
#include "device_util.hpp"
#include "moe_internal.hpp"

namespace tmt {

// Butterfly max / sum / arg-max over groups of EP lanes (xor offsets EP/2 .. 1).
template <int EP>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (EP >= 64) v = fmaxf(v, xor_lane<32>(v));
    if constexpr (EP >= 32) v = fmaxf(v, xor_lane<16>(v));
    if constexpr (EP >= 16) v = fmaxf(v, xor_lane<8>(v));
    v = fmaxf(v, xor_lane<4>(v));
    v = fmaxf(v, xor_lane<2>(v));
    v = fmaxf(v, xor_lane<1>(v));
    return v;
}
template <int EP>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (EP >= 64) v += xor_lane<32>(v);
    if constexpr (EP >= 32) v += xor_lane<16>(v);
    if constexpr (EP >= 16) v += xor_lane<8>(v);
    v += xor_lane<4>(v);
    v += xor_lane<2>(v);
    v += xor_lane<1>(v);
    return v;
}
// One arg-max step at offset OFF over (logit desc, expert asc).
template <int OFF>
__device__ __forceinline__ void argmax_step(float& bv, int& be) {
    const float ov = xor_lane<OFF>(bv);
    const int oe = xor_lane<OFF>(be);
    if (ov > bv || (ov == bv && oe < be)) {
        bv = ov;
        be = oe;
    }
}

// Softmax and top-k of one row held by EP lanes (lane e_mine = expert):
// softmax over the row (moe.cu:41-49); K rounds of a butterfly arg-max over
// (logit desc, expert asc), i.e. strict '>' with ties to the lower index
// (moe.cu:52-63); renormalised gate of pick j on lane j (moe.cu:64-66).
// Lanes out of a round (invalid or already picked) enter it as
// (-inf, e + 64), which every candidate beats. The winner's probability is
// recomputed from its logit with the operations its own lane used, so it
// equals that lane's value bit for bit without another exchange.
struct RowPick {
    float prob, lse, gate;
    int idx;
    bool sel;
};
template <int EP>
__device__ __forceinline__ RowPick softmax_topk(float logit, bool e_valid, int e_mine, int K) {
    RowPick o;
    const float lv = e_valid ? logit : -INFINITY;
    const float mx = group_max<EP>(lv);
    const float ex = e_valid ? __expf(lv - mx) : 0.0f;
    const float se = group_sum<EP>(ex);
    o.prob = ex / se;
    o.lse = mx + __logf(se);
    bool sel = false;
    int out_e = 0;
    float out_p = 0.0f, zsum = 0.0f;
    for (int j = 0; j < K; ++j) {
        const bool in = e_valid && !sel;
        float bv = in ? logit : -INFINITY;
        int be = in ? e_mine : e_mine + 64;
        if constexpr (EP >= 64) argmax_step<32>(bv, be);
        if constexpr (EP >= 32) argmax_step<16>(bv, be);
        if constexpr (EP >= 16) argmax_step<8>(bv, be);
        argmax_step<4>(bv, be);
        argmax_step<2>(bv, be);
        argmax_step<1>(bv, be);
        const float bp = __expf(bv - mx) / se;
        if (e_mine == be) sel = true;
        if (e_mine == j) {
            out_e = be;
            out_p = bp;
        }
        zsum += bp;
    }
    o.sel = sel;
    o.idx = out_e;
    o.gate = out_p / zsum;
    return o;
}

constexpr int kPairBatch = 4;  // expert dot products per wave with loads in flight

// Logits of token row `row` into s_logit[E]: wave w of nw computes experts
// w, w + nw, ..., each as the canonical lane partials (lane L owns the
// elements c*512 + 8L + t, fmaf in ascending k) and the full xor butterfly
// (32 .. 1), which adds the same partial trees as router_kernel's
// reduce-scatter, so the bits do not depend on nw. Two 512-element chunks
// per pass, with every load of the pass (and the bias) in flight together.
__device__ __forceinline__ void token_logits(const RouterParams& p, int row, float* s_logit, int wave, int nw,
                                             int lane) {
    const int E = p.E, d = p.d;
    const int nch = (d + 511) / 512;
    for (int e0 = wave; e0 < E; e0 += nw * kPairBatch) {
        float acc[kPairBatch], bias[kPairBatch];
#pragma unroll
        for (int u = 0; u < kPairBatch; ++u) {
            acc[u] = 0.0f;
            bias[u] = (p.bias != nullptr && e0 + nw * u < E) ? p.bias[e0 + nw * u] : 0.0f;
        }
        for (int c = 0; c < nch; c += 2) {
            int k[2];
            bool ok[2];
            uint4 wv[2][kPairBatch], xv[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                k[h] = (c + h) * 512 + lane * 8;
                ok[h] = k[h] < d;
                const int kk = ok[h] ? k[h] : 0;  // clamped: unused lanes load a valid address
#pragma unroll
                for (int u = 0; u < kPairBatch; ++u) {
                    const int e = min(e0 + nw * u, E - 1);  // clamped: extra pairs are discarded
                    wv[h][u] = *reinterpret_cast<const uint4*>(p.Wr + (int64_t)e * d + kk);
                }
                xv[h] = *reinterpret_cast<const uint4*>(p.X + (int64_t)row * d + kk);
            }
            // Branch-free (a lane past d keeps its partial by a select): loads
            // under a branch would be sunk there and waited for separately.
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float xf[8];
                unpack8(xv[h], xf);
#pragma unroll
                for (int u = 0; u < kPairBatch; ++u) {
                    float wf[8];
                    unpack8(wv[h][u], wf);
                    float a = acc[u];
#pragma unroll
                    for (int t = 0; t < 8; ++t) a = __builtin_fmaf(xf[t], wf[t], a);
                    acc[u] = ok[h] ? a : acc[u];
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kPairBatch; ++u) {
            float v = acc[u];
            v += xor_lane<32>(v);
            v += xor_lane<16>(v);
            v += xor_lane<8>(v);
            v += xor_lane<4>(v);
            v += xor_lane<2>(v);
            v += xor_lane<1>(v);
            const int e = e0 + nw * u;
            if (lane == 0 && e < E) s_logit[e] = p.bias != nullptr ? v + bias[u] : v;
        }
    }
}

// T == 1: the whole dispatch from wave 0's registers after the softmax. A
// single token's K picks are distinct experts with one slot each, taken in
// ascending expert order, so counts, offsets, slots and the expert order
// are ballots over the picked lanes.
template <int EP>
__device__ __forceinline__ void one_token_dispatch(const RouterParams& p, const ScanParams& sp,
                                                   const PermuteParams& pp, float logit, bool ev,
                                                   const RowPick& pk, int lane) {
    const int E = p.E, K = p.K;
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    const bool picked = ev && pk.sel;
    const uint64_t selm = __ballot(picked);
    const uint64_t valm = __ballot(ev);
    const int off = __popcll(selm & below);
    const int ord = picked ? off : K + __popcll(valm & ~selm & below);
    const int pj = pk.idx;  // pick j on lane j < K
    const int slot = __popcll(selm & (pj == 0 ? 0ull : (~0ull >> (64 - pj))));
    // Switch aux (moe.cu:456-465) with T = 1: E * sum_e p_e * (c_e / K).
    const float inv_tk = 1.0f / (float)K;
    const float aux = group_sum<EP>(picked ? pk.prob * inv_tk : 0.0f) * (float)E;
    if (lane < E) {
        p.logits[lane] = logit;
        p.probs[lane] = pk.prob;
        sp.offsets[lane] = off;
        sp.counts[lane] = picked ? 1 : 0;
        reinterpret_cast<int32_t*>(sp.stats + 2)[lane] = picked ? 1 : 0;
        sp.order[ord] = lane;
    }
    if (lane < K) {
        p.idx[lane] = pj;
        p.gate[lane] = pk.gate;
        pp.perm[lane] = 0;
        pp.slot_of[lane] = slot;
    }
    if (lane == 0) {
        p.lse[0] = pk.lse;
        sp.offsets[E] = K;
        sp.stats[0] = aux;
        sp.stats[1] = pk.lse * pk.lse;  // z-loss mean (moe.cu:268-278)
    }
}

}  // namespace tmt
