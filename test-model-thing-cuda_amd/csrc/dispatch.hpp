// dispatch.hpp -- decode-batch dispatch computed from the [T][topk] pick
// table inside the kernels that consume it (T <= kSkinnyMaxTokens).
//
// The dispatch (tmt-cuda/src/moe.cu:97-115: per-expert counts, offsets by an
// exclusive scan, each pick given a slot in its expert's segment -- here in
// token order, as everywhere in this library, rather than the reference's
// atomic order) is a pure function of the picks. For a
// decode batch every consumer holds the whole table in one wave's registers
// (at most 512 picks: eight per lane) and derives what it needs with ballots:
// an expert's first slot and row count, or one pick's slot. That replaces the
// router's cross-block handoff, which on this GPU pays a device-scope release
// and acquire (L2 write-back and invalidate) in every router block.
#pragma once
#include "moe_internal.hpp"

namespace tmt {

constexpr int kPickGroups = kSkinnyMaxTokens * kMaxTopK / 64;

// Entries q * 64 + lane of the pick table (-1 past `slots`, or without a
// table: E == 1, where slot == token).
__device__ __forceinline__ void load_pick_table(const int32_t* idx, int slots, int lane, int (&ent)[kPickGroups]) {
#pragma unroll
    for (int q = 0; q < kPickGroups; ++q) {
        const int i = q * 64 + lane;
        ent[q] = (idx != nullptr && i < slots) ? idx[i] : -1;
    }
}

// Expert e's first slot (picks of lower experts) and row count.
__device__ __forceinline__ void expert_span(const int (&ent)[kPickGroups], int slots, int e, int& row0, int& rows) {
    int below = 0, mine = 0;
#pragma unroll
    for (int q = 0; q < kPickGroups; ++q) {
        if (q * 64 >= slots) break;  // uniform
        below += __popcll(__ballot(ent[q] >= 0 && ent[q] < e));
        mine += __popcll(__ballot(ent[q] == e));
    }
    row0 = below;
    rows = mine;
}

// Slot of pick i (wave-uniform) whose expert is e (wave-uniform): the picks
// of lower experts, then expert e's picks of lower index (= earlier tokens).
__device__ __forceinline__ int pick_slot(const int (&ent)[kPickGroups], int slots, int e, int i, int lane) {
    int n = 0;
#pragma unroll
    for (int q = 0; q < kPickGroups; ++q) {
        if (q * 64 >= slots) break;  // uniform
        const int k = q * 64 + lane;
        n += __popcll(__ballot(ent[q] >= 0 && (ent[q] < e || (ent[q] == e && k < i))));
    }
    return n;
}


// One wave: every table the router's last block writes otherwise
// (route_small_kernel) -- counts and offsets (lane e), the processing order,
// each pick's slot, and the Switch aux / z statistics. EP >= E is a power of
// two: the per-expert loops are unrolled to EP, so that their ballots are
// independent instructions rather than a chain of dependent scalar steps
// (one wave alone on its CU has nothing to hide such a chain behind).
template <int EP>
__device__ __forceinline__ void write_dispatch_ep(const DispatchTables& t, const int (&ent)[kPickGroups], int lane) {
    const int E = t.E, K = t.K, T = t.T, slots = T * K;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    // Each pick's rank among its expert's picks (pick order = token order)
    // and the per-expert running counts, group by group.
    int run[EP];
#pragma unroll
    for (int e = 0; e < EP; ++e) run[e] = 0;
    int rel[kPickGroups];
#pragma unroll
    for (int q = 0; q < kPickGroups; ++q) {
        rel[q] = 0;
        if (q * 64 < slots) {  // uniform
            const int v = ent[q];
            int r = 0;
#pragma unroll
            for (int e = 0; e < EP; ++e) {
                const uint64_t mk = __ballot(v == e);
                r = v == e ? run[e] + __popcll(mk & lt) : r;
                run[e] += __popcll(mk);
            }
            rel[q] = r;
        }
    }
    int cnt = 0;
#pragma unroll
    for (int e = 0; e < EP; ++e) cnt = lane == e ? run[e] : cnt;
    int incl = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o, 64);
        if (lane >= o) incl += v;
    }
    const int off = incl - cnt;
    int ord = 0;
#pragma unroll
    for (int e = 0; e < EP; ++e) ord += e < E && ((run[e] > cnt) || (run[e] == cnt && e < lane));
    int pos[kPickGroups];
#pragma unroll
    for (int q = 0; q < kPickGroups; ++q) pos[q] = __shfl(off, ent[q] < 0 ? 0 : ent[q], 64) + rel[q];

    // Probability column sums: lane l adds rows l / EP, l / EP + 64 / EP, ...
    // of expert l % EP, then the 64 / EP partials of an expert are added
    // pairwise; sum of lse^2 by a butterfly over lane r = row r.
    constexpr int RP = 64 / EP;  // row phases
    const int ce = lane % EP, rp = lane / EP;
    float pv[kSkinnyMaxTokens / RP];
#pragma unroll
    for (int k = 0; k < kSkinnyMaxTokens / RP; ++k) {
        const int r = rp + k * RP;
        pv[k] = t.probs[(int64_t)min(r, T - 1) * E + min(ce, E - 1)];
    }
    const float lv = t.lse[min(lane, T - 1)];
    float fs = 0.0f;
#pragma unroll
    for (int k = 0; k < kSkinnyMaxTokens / RP; ++k)
        if (rp + k * RP < T) fs += pv[k];
#pragma unroll
    for (int o = EP; o < 64; o <<= 1) fs += __shfl_xor(fs, o, 64);
    float l2 = lane < T ? lv * lv : 0.0f;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) l2 += __shfl_xor(l2, o, 64);
    // aux = E * sum_e (P_e / T) (c_e / (T K)) on lane 0
    const float inv_t = 1.0f / (float)T;
    const float inv_tk = 1.0f / ((float)T * (float)K);
    float a = lane < E ? (fs * inv_t) * ((float)cnt * inv_tk) : 0.0f;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) a += __shfl_xor(a, o, 64);

#pragma unroll
    for (int q = 0; q < kPickGroups; ++q) {
        const int i = q * 64 + lane;
        if (i < slots) {
            t.perm[pos[q]] = i / K;
            t.slot_of[i] = pos[q];
        }
    }
    if (lane < E) {
        t.offsets[lane] = off;
        t.counts[lane] = cnt;
        t.order[ord] = lane;
        reinterpret_cast<int32_t*>(t.stats + 2)[lane] = cnt;
    }
    if (lane == 0) {
        t.offsets[E] = slots;
        t.stats[0] = a * (float)E;
        t.stats[1] = l2 * inv_t;
    }
}

__device__ __forceinline__ void write_dispatch(const DispatchTables& t, const int (&ent)[kPickGroups], int lane) {
    if (t.E <= 8) write_dispatch_ep<8>(t, ent, lane);
    else if (t.E <= 16) write_dispatch_ep<16>(t, ent, lane);
    else if (t.E <= 32) write_dispatch_ep<32>(t, ent, lane);
    else write_dispatch_ep<64>(t, ent, lane);
}

}  // namespace tmt
