// router.hip -- router, expert histogram, offset scan and stable permutation.
//
// Replaces the reference's router_topk_kernel / topk_kernel / count_kernel /
// fill_kernel and the host-side offset computation (tmt-cuda/src/moe.cu:10-115,
// 404-424). Differences by design:
//  * logits use one canonical fp32 summation order (lane partials + xor
//    butterfly) that the host oracle reproduces bit for bit, for any E <= 64;
//  * top-k compares logits (same order as the probabilities) with ties going
//    to the lower expert index, as the reference's strict '>' scan does;
//  * counts, offsets and the permutation never leave the device, and the
//    permutation is stable (ascending token inside each expert segment)
//    instead of atomic-order (moe.cu:103-115).
#include "device_util.hpp"
#include "moe_internal.hpp"

namespace tmt {

// Expert lanes per row: E rounded up to a power of two, at least 8 so that a
// wave holds at most 8 rows (64 partial sums per lane, no register spills).
int router_ep(int E) {
    int ep = 8;
    while (ep < E) ep <<= 1;
    return ep;
}
int router_rows_per_wave(int E) { return 64 / router_ep(E); }

// One wave routes R = 64/EP rows at a time. Lane L owns the elements
// k = c*512 + 8L + t of each row (t = 0..7, chunk c = 0, 1, ...), and keeps
// one fp32 partial per (row, expert), accumulated with fmaf in ascending k.
// A reduce-scatter xor butterfly (offsets 32..1) then leaves lane l with the
// full dot product of row l/EP and expert l%EP; each addition pairs the same
// partial trees as the full butterfly, so the bits equal the canonical order.
template <int EP>
__global__ __launch_bounds__(kThreads) void router_kernel(RouterParams p) {
    constexpr int R = 64 / EP;
    extern __shared__ uint4 smem_w[];  // Wr [E][d] bf16
    __shared__ int s_cnt[kMaxExperts];
    __shared__ float s_stat[4][kMaxExperts + 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int d = p.d, E = p.E, K = p.K;
    {
        const uint4* src = reinterpret_cast<const uint4*>(p.Wr);
        const int nvec = E * d / 8;
        for (int i = tid; i < nvec; i += kThreads) smem_w[i] = src[i];
    }
    if (tid < kMaxExperts) s_cnt[tid] = 0;
    __syncthreads();
    const uint16_t* wl = reinterpret_cast<const uint16_t*>(smem_w);

    const int row_begin = blockIdx.x * p.rows_per_block;
    const int row_end = min(p.T, row_begin + p.rows_per_block);
    const int e_mine = lane % EP;
    const int r_mine = lane / EP;
    const bool e_valid = e_mine < E;
    const int nch = (d + 511) / 512;
    float psum = 0.0f, lsum = 0.0f;

    for (int r0 = row_begin + wave * R; r0 < row_end; r0 += 4 * R) {
        float acc[R * EP];
#pragma unroll
        for (int i = 0; i < R * EP; ++i) acc[i] = 0.0f;

        for (int c = 0; c < nch; ++c) {
            const int k0 = c * 512 + lane * 8;
            if (k0 >= d) continue;  // this lane owns no element of the chunk
            float xf[R][8];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = r0 + r;
                uint4 xv = make_uint4(0, 0, 0, 0);
                if (row < row_end)
                    xv = *reinterpret_cast<const uint4*>(p.X + (int64_t)row * d + k0);
                unpack8(xv, xf[r]);
            }
#pragma unroll
            for (int e = 0; e < EP; ++e) {
                if (e < E) {
                    float wf[8];
                    unpack8(*reinterpret_cast<const uint4*>(wl + e * d + k0), wf);
#pragma unroll
                    for (int r = 0; r < R; ++r)
#pragma unroll
                        for (int t = 0; t < 8; ++t)
                            acc[r * EP + e] = __builtin_fmaf(xf[r][t], wf[t], acc[r * EP + e]);
                }
            }
        }

        // Reduce-scatter butterfly: at offset `off` the lane keeps the half of
        // its entries whose bit log2(off) equals its own lane bit.
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const bool upper = (lane & off) != 0;
#pragma unroll
            for (int t = 0; t < off; ++t) {
                const float lo = acc[t], hi = acc[t + off];
                const float send = upper ? lo : hi;
                const float keep = upper ? hi : lo;
                const float recv = shfl_xor(send, off);
                acc[t] = keep + recv;
            }
        }
        float logit = acc[0];
        if (p.bias != nullptr && e_valid) logit = logit + p.bias[e_mine];

        const int row = r0 + r_mine;
        const bool row_valid = row < row_end;

        // Softmax over the EP lanes of this row (moe.cu:41-49).
        const float lv = e_valid ? logit : -INFINITY;
        float mx = lv;
#pragma unroll
        for (int off = EP / 2; off >= 1; off >>= 1) mx = fmaxf(mx, shfl_xor(mx, off));
        const float ex = e_valid ? __expf(lv - mx) : 0.0f;
        float se = ex;
#pragma unroll
        for (int off = EP / 2; off >= 1; off >>= 1) se += shfl_xor(se, off);
        const float prob = ex / se;
        const float lse = mx + __logf(se);

        // Top-k: K rounds of a butterfly argmax over (logit desc, expert asc).
        bool sel = false;
        int out_e = 0;
        float out_p = 0.0f, zsum = 0.0f;
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j) {
            if (j < K) {
                bool has = e_valid && !sel;
                float bv = logit, bp = prob;
                int be = e_mine;
#pragma unroll
                for (int off = EP / 2; off >= 1; off >>= 1) {
                    const float ov = shfl_xor(bv, off);
                    const float op = shfl_xor(bp, off);
                    const int oe = shfl_xor(be, off);
                    const int oh = shfl_xor((int)has, off);
                    const bool take = oh && (!has || ov > bv || (ov == bv && oe < be));
                    if (take) { bv = ov; bp = op; be = oe; has = true; }
                }
                if (e_mine == be) sel = true;
                if (e_mine == j) { out_e = be; out_p = bp; }
                zsum += bp;
            }
        }

        if (row_valid) {
            if (e_valid) {
                p.logits[(int64_t)row * E + e_mine] = logit;
                p.probs[(int64_t)row * E + e_mine] = prob;
                psum += prob;
            }
            if (e_mine < K) {
                p.idx[(int64_t)row * K + e_mine] = out_e;
                p.gate[(int64_t)row * K + e_mine] = out_p / zsum;
            }
            if (e_mine == 0) {
                p.lse[row] = lse;
                lsum += lse * lse;
            }
            if (sel) atomicAdd(&s_cnt[e_mine], 1);
        }
    }

    // Block statistics in a fixed order: row slots (xor butterfly), then waves.
#pragma unroll
    for (int off = 32; off >= EP; off >>= 1) {
        psum += shfl_xor(psum, off);
        lsum += shfl_xor(lsum, off);
    }
    if (lane < EP) s_stat[wave][lane] = psum;
    if (lane == 0) s_stat[wave][kMaxExperts] = lsum;
    __syncthreads();
    const int b = blockIdx.x;
    if (tid < E) {
        p.blkstat[(int64_t)b * (E + 1) + tid] =
            ((s_stat[0][tid] + s_stat[1][tid]) + s_stat[2][tid]) + s_stat[3][tid];
        p.blkcnt[(int64_t)b * E + tid] = s_cnt[tid];
    }
    if (tid == 0)
        p.blkstat[(int64_t)b * (E + 1) + E] =
            ((s_stat[0][kMaxExperts] + s_stat[1][kMaxExperts]) + s_stat[2][kMaxExperts]) +
            s_stat[3][kMaxExperts];
}

hipError_t launch_router(const RouterParams& p, int nblk, hipStream_t s) {
    const size_t lds = (size_t)p.E * p.d * 2;
    const int ep = router_ep(p.E);
    dim3 grid(nblk), block(kThreads);
    switch (ep) {
        case 8: router_kernel<8><<<grid, block, lds, s>>>(p); break;
        case 16: router_kernel<16><<<grid, block, lds, s>>>(p); break;
        case 32: router_kernel<32><<<grid, block, lds, s>>>(p); break;
        case 64: router_kernel<64><<<grid, block, lds, s>>>(p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Single workgroup: per-expert totals, exclusive offsets, per-block bases,
// the aux / z statistics and the descending-count expert order. Every sum is
// taken in a fixed order, so the statistics are run-to-run deterministic.
__global__ __launch_bounds__(1024) void scan_kernel(ScanParams p) {
    __shared__ int s_seg[1024];
    __shared__ float s_fseg[1024];
    __shared__ int s_off[kMaxExperts + 1];
    __shared__ int s_cnt[kMaxExperts];
    __shared__ float s_fsum[kMaxExperts + 1];
    const int tid = threadIdx.x;
    const int E = p.E, nblk = p.nblk;

    // 1) per (segment, expert) sums of the block histograms
    const int S = 1024 / E;
    const int chunk = (nblk + S - 1) / S;
    if (tid < S * E) {
        const int e = tid % E, seg = tid / E;
        const int b0 = seg * chunk, b1 = min(nblk, b0 + chunk);
        int sum = 0;
        for (int b = b0; b < b1; ++b) sum += p.blkcnt[(int64_t)b * E + e];
        s_seg[seg * E + e] = sum;
    }
    // 1b) per (segment, statistic) sums of the block statistics
    const int E1 = E + 1;
    const int S2 = 1024 / E1;
    const int chunk2 = (nblk + S2 - 1) / S2;
    if (tid < S2 * E1) {
        const int q = tid % E1, seg = tid / E1;
        const int b0 = seg * chunk2, b1 = min(nblk, b0 + chunk2);
        float sum = 0.0f;
        for (int b = b0; b < b1; ++b) sum += p.blkstat[(int64_t)b * E1 + q];
        s_fseg[seg * E1 + q] = sum;
    }
    __syncthreads();
    // 2) exclusive scan over segments, per expert
    if (tid < E) {
        int run = 0;
        for (int seg = 0; seg < S; ++seg) {
            const int c = s_seg[seg * E + tid];
            s_seg[seg * E + tid] = run;
            run += c;
        }
        s_cnt[tid] = run;
    }
    if (tid < E1) {
        float run = 0.0f;
        for (int seg = 0; seg < S2; ++seg) run += s_fseg[seg * E1 + tid];
        s_fsum[tid] = run;
    }
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int e = 0; e < E; ++e) {
            s_off[e] = run;
            run += s_cnt[e];
        }
        s_off[E] = run;
        // Switch aux (moe.cu:456-465) and z-loss mean (moe.cu:268-278).
        float aux = 0.0f, z = 0.0f;
        if (p.T > 0) {
            const float inv_t = 1.0f / (float)p.T;
            const float inv_tk = 1.0f / ((float)p.T * (float)p.K);
            for (int e = 0; e < E; ++e) aux += (s_fsum[e] * inv_t) * ((float)s_cnt[e] * inv_tk);
            aux *= (float)E;
            z = s_fsum[E] * inv_t;
        }
        p.stats[0] = aux;
        p.stats[1] = z;
    }
    __syncthreads();
    if (tid <= E) p.offsets[tid] = s_off[tid];
    if (tid < E) {
        p.counts[tid] = s_cnt[tid];
        reinterpret_cast<int32_t*>(p.stats + 2)[tid] = s_cnt[tid];
        int rank = 0;
        for (int e = 0; e < E; ++e)
            rank += (s_cnt[e] > s_cnt[tid]) || (s_cnt[e] == s_cnt[tid] && e < tid);
        p.order[rank] = tid;
    }
    // 3) per-block bases
    if (tid < S * E) {
        const int e = tid % E, seg = tid / E;
        const int b0 = seg * chunk, b1 = min(nblk, b0 + chunk);
        int run = s_off[e] + s_seg[seg * E + e];
        for (int b = b0; b < b1; ++b) {
            p.blkbase[(int64_t)b * E + e] = run;
            run += p.blkcnt[(int64_t)b * E + e];
        }
    }
}

hipError_t launch_scan(const ScanParams& p, hipStream_t s) {
    scan_kernel<<<1, 1024, 0, s>>>(p);
    return hipGetLastError();
}

// Stable permutation. Inside a block the (token, j) pairs are processed in
// groups of 64 lanes (floor(64/K) tokens each); a ballot per expert gives
// each pair its rank among earlier pairs of the group with the same expert.
// Group bases come from an in-LDS scan over the block's groups on top of the
// block base from scan_kernel, so slots follow ascending token order.
constexpr int kMaxGroups = 64;

__global__ __launch_bounds__(kThreads) void permute_kernel(PermuteParams p) {
    __shared__ int s_g[kMaxGroups][kMaxExperts];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = p.K, E = p.E;
    const int RG = 64 / K;
    const int pairs = RG * K;
    const int row_begin = blockIdx.x * p.rows_per_block;
    const int row_end = min(p.T, row_begin + p.rows_per_block);
    const int G = (row_end - row_begin + RG - 1) / RG;
    const int rr = lane / K, j = lane % K;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));

    for (int g = wave; g < G; g += 4) {
        const int row = row_begin + g * RG + rr;
        const bool valid = lane < pairs && row < row_end;
        const int e = valid ? p.idx[(int64_t)row * K + j] : -1;
        for (int ee = 0; ee < E; ++ee) {
            const uint64_t m = __ballot(e == ee);
            if (lane == ee) s_g[g][ee] = __popcll(m);
        }
    }
    __syncthreads();
    if (tid < E) {
        int run = p.blkbase[(int64_t)blockIdx.x * E + tid];
        for (int g = 0; g < G; ++g) {
            const int c = s_g[g][tid];
            s_g[g][tid] = run;
            run += c;
        }
    }
    __syncthreads();
    for (int g = wave; g < G; g += 4) {
        const int row = row_begin + g * RG + rr;
        const bool valid = lane < pairs && row < row_end;
        const int e = valid ? p.idx[(int64_t)row * K + j] : -1;
        int rank = 0;
        for (int ee = 0; ee < E; ++ee) {
            const uint64_t m = __ballot(e == ee);
            if (e == ee) rank = __popcll(m & lt_mask);
        }
        if (valid) {
            const int pos = s_g[g][e] + rank;
            p.perm[pos] = row;
            p.slot_of[(int64_t)row * K + j] = pos;
        }
    }
}

hipError_t launch_permute(const PermuteParams& p, int nblk, hipStream_t s) {
    const int RG = 64 / p.K;
    if ((p.rows_per_block + RG - 1) / RG > kMaxGroups) return hipErrorInvalidValue;
    permute_kernel<<<nblk, kThreads, 0, s>>>(p);
    return hipGetLastError();
}

__global__ __launch_bounds__(kThreads) void dense_dispatch_kernel(
    int T, int32_t* perm, int32_t* slot_of, float* gate, int32_t* counts,
    int32_t* offsets, int32_t* order, float* stats) {
    const int r = blockIdx.x * kThreads + threadIdx.x;
    if (r < T) {
        perm[r] = r;
        slot_of[r] = r;
        gate[r] = 1.0f;
    }
    if (r == 0) {
        counts[0] = T;
        offsets[0] = 0;
        offsets[1] = T;
        order[0] = 0;
        stats[0] = 0.0f;
        stats[1] = 0.0f;
        reinterpret_cast<int32_t*>(stats + 2)[0] = T;
    }
}

hipError_t launch_dense_dispatch(int T, int32_t* perm, int32_t* slot_of,
                                 float* gate, int32_t* counts, int32_t* offsets,
                                 int32_t* order, float* stats, hipStream_t s) {
    const int grid = T > 0 ? (T + kThreads - 1) / kThreads : 1;
    dense_dispatch_kernel<<<grid, kThreads, 0, s>>>(T, perm, slot_of, gate, counts,
                                                    offsets, order, stats);
    return hipGetLastError();
}

}  // namespace tmt
