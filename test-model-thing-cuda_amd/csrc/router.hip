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
#include "ln_row.hpp"
#include "moe_internal.hpp"
#include "route_row.hpp"

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
// Stage Wr [E][d] (bf16) in LDS: all of a thread's 16-byte loads are issued
// before any of them is stored, so the fill costs one memory round trip.
__device__ __forceinline__ void stage_router_weights(const uint16_t* Wr, int nvec, uint4* dst) {
    const uint4* src = reinterpret_cast<const uint4*>(Wr);
    constexpr int kBatch = 8;
    const int nt = (int)blockDim.x;
    for (int base = threadIdx.x; base < nvec; base += kBatch * nt) {
        uint4 v[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int j = min(base + i * nt, nvec - 1);  // clamped: no load under a branch
            v[i] = src[j];
        }
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int j = base + i * nt;
            if (j < nvec) dst[j] = v[i];
        }
    }
}

// Route rows [row_begin, row_end) with the block's 4 waves: logits, probs,
// top-k indices and gates, lse. Per-expert pick counts are added to s_cnt
// (LDS atomics); each wave leaves its sum of probabilities per expert in
// s_stat[wave][e] and its sum of lse^2 in s_stat[wave][kMaxExperts]. When
// s_idx is given, the picks are also stored there ([row - row_begin][j]).
// Reduce-scatter level at offset OFF over the first 2*OFF entries of acc:
// afterwards acc[t] (t < OFF) holds, on lane l, the sum of the entry the lane
// keeps (t, or t + OFF when bit OFF of l is set) and its partner's copy of
// that entry. OFF = 32 / 16 use the row-swap instructions, which deliver
// both operands of every addition without a select.
template <int OFF>
__device__ __forceinline__ void reduce_scatter_level(float* acc, int lane) {
    if constexpr (OFF >= 16) {
#pragma unroll
        for (int t = 0; t < OFF; ++t) {
            const u32x2_t sw = OFF == 32
                ? __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[t]), __float_as_uint(acc[t + OFF]), false, false)
                : __builtin_amdgcn_permlane16_swap(__float_as_uint(acc[t]), __float_as_uint(acc[t + OFF]), false, false);
            // lanes without bit OFF: {own lo, partner lo}; with it: {partner hi, own hi}
            acc[t] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
    } else {
        const bool upper = (lane & OFF) != 0;
#pragma unroll
        for (int t = 0; t < OFF; ++t) {
            const float lo = acc[t], hi = acc[t + OFF];
            const float send = upper ? lo : hi;
            const float keep = upper ? hi : lo;
            acc[t] = keep + xor_lane<OFF>(send);
        }
    }
}

// NCH > 0: the rows are the block input S and pass through the LayerNorm
// first (ln_row.hpp, the same arithmetic as ln_fwd_kernel): the wave loads
// its R rows whole (NCH chunks of 512 elements), writes H and the row
// statistics, and computes the logits from H as rounded to bf16, as the
// router would read it back.
template <int EP, int NW, int NCH = 0>
__device__ __forceinline__ void route_rows(const RouterParams& p, const uint16_t* wl, int row_begin,
                                           int row_end, int* s_cnt,
                                           float (*s_stat)[kMaxExperts + 1], int* s_idx) {
    constexpr int R = 64 / EP;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int d = p.d, E = p.E, K = p.K;
    const int e_mine = lane % EP;
    const int r_mine = lane / EP;
    const bool e_valid = e_mine < E;
    const int nch = (d + 511) / 512;
    float psum = 0.0f, lsum = 0.0f;

    for (int r0 = row_begin + wave * R; r0 < row_end; r0 += NW * R) {
        float acc[R * EP];
#pragma unroll
        for (int i = 0; i < R * EP; ++i) acc[i] = 0.0f;

        uint4 hv[R][NCH > 0 ? NCH : 1];  // LayerNorm: the rows' H pieces
        if constexpr (NCH > 0) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int c = 0; c < NCH; ++c) {
                    const int row = r0 + r, k0 = c * 512 + lane * 8;
                    hv[r][c] = make_uint4(0, 0, 0, 0);
                    if (row < row_end && k0 < d) hv[r][c] = *reinterpret_cast<const uint4*>(p.X + (int64_t)row * d + k0);
                }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = r0 + r;
                float ls = 0.0f, lq = 0.0f;
#pragma unroll
                for (int c = 0; c < NCH; ++c) {
                    if (c * 512 + lane * 8 < d) {
                        float v[8];
                        unpack8(hv[r][c], v);
                        ln_accumulate(v, ls, lq);
                    }
                }
                float mean, rstd;
                ln_finish(ls, lq, d, mean, rstd);
#pragma unroll
                for (int c = 0; c < NCH; ++c) {
                    const int k0 = c * 512 + lane * 8;
                    if (k0 < d) {
                        float v[8];
                        unpack8(hv[r][c], v);
                        hv[r][c] = ln_apply8(v, mean, rstd, p.ln_gamma, p.ln_beta, k0);
                        if (row < row_end) *reinterpret_cast<uint4*>(p.ln_H + (int64_t)row * d + k0) = hv[r][c];
                    }
                }
                if (lane == 0 && row < row_end) {
                    p.ln_mean[row] = mean;
                    p.ln_rstd[row] = rstd;
                }
            }
        }
        // Logit partials of chunk c (k0 = c * 512 + 8 * lane < d) from the
        // rows' elements xf.
        auto dots = [&](int k0, const float (&xf)[R][8]) {
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
        };
        if constexpr (NCH > 0) {
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const int k0 = c * 512 + lane * 8;
                if (k0 < d) {
                    float xf[R][8];
#pragma unroll
                    for (int r = 0; r < R; ++r) unpack8(hv[r][c], xf[r]);
                    dots(k0, xf);
                }
            }
        } else {
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
                dots(k0, xf);
            }
        }

        // Reduce-scatter butterfly: at offset `off` the lane keeps the half of
        // its entries whose bit log2(off) equals its own lane bit.
        reduce_scatter_level<32>(acc, lane);
        reduce_scatter_level<16>(acc, lane);
        reduce_scatter_level<8>(acc, lane);
        reduce_scatter_level<4>(acc, lane);
        reduce_scatter_level<2>(acc, lane);
        reduce_scatter_level<1>(acc, lane);
        float logit = acc[0];
        if (p.bias != nullptr && e_valid) logit = logit + p.bias[e_mine];

        const int row = r0 + r_mine;
        const bool row_valid = row < row_end;

        const RowPick pk = softmax_topk<EP>(logit, e_valid, e_mine, K);
        const float prob = pk.prob, lse = pk.lse;
        const bool sel = pk.sel;

        if (row_valid) {
            if (e_valid) {
                p.logits[(int64_t)row * E + e_mine] = logit;
                p.probs[(int64_t)row * E + e_mine] = prob;
                psum += prob;
            }
            if (e_mine < K) {
                p.idx[(int64_t)row * K + e_mine] = pk.idx;
                p.gate[(int64_t)row * K + e_mine] = pk.gate;
                if (s_idx) s_idx[(row - row_begin) * K + e_mine] = pk.idx;
            }
            if (e_mine == 0) {
                p.lse[row] = lse;
                lsum += lse * lse;
            }
            if (sel) atomicAdd(&s_cnt[e_mine], 1);
        }
    }

    // Per-wave statistics in a fixed order: row slots (xor butterfly).
    if constexpr (EP <= 32) { psum += xor_lane<32>(psum); lsum += xor_lane<32>(lsum); }
    if constexpr (EP <= 16) { psum += xor_lane<16>(psum); lsum += xor_lane<16>(lsum); }
    if constexpr (EP <= 8) { psum += xor_lane<8>(psum); lsum += xor_lane<8>(lsum); }
    if (lane < EP) s_stat[wave][lane] = psum;
    if (lane == 0) s_stat[wave][kMaxExperts] = lsum;
}

// One wave routes R = 64/EP rows at a time. Lane L owns the elements
// k = c*512 + 8L + t of each row (t = 0..7, chunk c = 0, 1, ...), and keeps
// one fp32 partial per (row, expert), accumulated with fmaf in ascending k.
// A reduce-scatter xor butterfly (offsets 32..1) then leaves lane l with the
// full dot product of row l/EP and expert l%EP; each addition pairs the same
// partial trees as the full butterfly, so the bits equal the canonical order.
// WLDS: Wr is staged in LDS (E*d*2 <= kRouterWrLdsBytes); otherwise the
// waves read it from global memory (it stays in L2), with the same
// arithmetic and therefore the same bits.
// NW waves per workgroup share one staged copy of Wr; the block statistics
// add the waves' sums in wave order.
// NCH > 0: the LayerNorm in front of the router is computed here (route_rows).
template <int EP, bool WLDS, int NW, int NCH>
__global__ __launch_bounds__(64 * NW) void router_kernel(RouterParams p) {
    extern __shared__ uint4 smem_w[];  // Wr [E][d] bf16 (WLDS)
    __shared__ int s_cnt[kMaxExperts];
    __shared__ float s_stat[NW][kMaxExperts + 1];

    const int tid = threadIdx.x;
    const int E = p.E;
    if constexpr (WLDS) stage_router_weights(p.Wr, E * p.d / 8, smem_w);
    if (tid < kMaxExperts) s_cnt[tid] = 0;
    __syncthreads();

    const int row_begin = blockIdx.x * p.rows_per_block;
    const int row_end = min(p.T, row_begin + p.rows_per_block);
    const uint16_t* wl = WLDS ? reinterpret_cast<const uint16_t*>(smem_w) : p.Wr;
    route_rows<EP, NW, NCH>(p, wl, row_begin, row_end, s_cnt, s_stat, nullptr);
    __syncthreads();
    // Block statistics: waves added in order.
    const int b = blockIdx.x;
    if (tid <= E) {
        const int col = tid < E ? tid : kMaxExperts;
        float v = s_stat[0][col];
#pragma unroll
        for (int w = 1; w < NW; ++w) v += s_stat[w][col];
        p.blkstat[(int64_t)b * (E + 1) + tid] = v;
        if (tid < E) p.blkcnt[(int64_t)b * E + tid] = s_cnt[tid];
    }
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

// ---- router logits on the matrix cores -----------------------------------
// Large routed batches without the LayerNorm (E <= 32): one 4-wave block per
// CU walks 128-row groups; wave w takes rows 32w .. 32w + 31 of a group and
// computes their logits with v_mfma_f32_32x32x16_bf16 (X rows as the A
// operand, Wr rows as B, fp32 accumulation), together with
// A = sum_k |x_k w_k| from a second MFMA over the operands with their sign
// bits cleared. Wr sits in LDS for the block (rows padded by 16 bytes); X
// streams through a per-wave double buffer in LDS in 128-element chunks,
// loaded as 4 rows x 256 bytes per instruction (the MFMA's own layout, 32
// rows x 32 bytes per instruction, kept the CU's load path busy for 37 us
// per block at c3), and on from one group into the next.
// The MFMA sums the same exact bf16 products as the canonical order does,
// only in another order, so a logit differs from the canonical one by at
// most
//   delta = (4 (5d/64 + 24) A + 8 (|logit| + |bias|)) u,  u = 2^-24,
// for every expert of the row: the canonical order rounds each product at
// most d/64 + 6 times before the bias, the MFMA path at most d/16 + 16
// times even with truncating arithmetic (twice the error per rounding),
// and the factor 4 covers both with room. Where the MFMA logits of the
// top K + 1 picks are more than 2 delta apart, the canonical logits rank the
// experts the same way, so the picks, their order and everything built from
// them (counts, offsets, permutation) are exactly the canonical router's;
// the row keeps the MFMA logits, and probabilities, lse and gates computed
// from them (within a few ulp of the canonical ones). A row with a closer
// pair, or with a non-finite value, is flagged and recomputed in the
// canonical order (the lane partials and full butterfly of token_logits,
// then softmax_topk): bit for bit what router_kernel writes. Flagged rows
// are taken in ascending row order, so the block statistics are
// deterministic.
// Sums of N entries per lane over the wave's 64 lanes (xor butterfly,
// offsets 32 .. 1) as a reduce-scatter: at offset OFF while n > 1 entries are
// left, the lanes with bit OFF set keep the upper half of their entries,
// adding their partner's copy, so lane l ends with entry
// sum_j bit(5 - j, l) * N / 2^(j+1) (j < log2 N); then plain butterfly steps.
// Every addition is own + partner of the same partial trees as the full
// butterfly, so each sum has that butterfly's bits.
template <int OFF, int N>
__device__ __forceinline__ void rs_sum_level(float* a, int lane) {
    if constexpr (N > 1) {
        const bool upper = (lane & OFF) != 0;
#pragma unroll
        for (int t = 0; t < N / 2; ++t) {
            const float lo = a[t], hi = a[t + N / 2];
            const float send = upper ? lo : hi;
            const float keep = upper ? hi : lo;
            a[t] = keep + xor_lane<OFF>(send);
        }
        rs_sum_level<OFF / 2, N / 2>(a, lane);
    } else if constexpr (OFF >= 1) {
        a[0] = a[0] + xor_lane<OFF>(a[0]);
        rs_sum_level<OFF / 2, 1>(a, lane);
    }
}
template <int N>
__device__ __forceinline__ int rs_sum_entry(int lane) {
    int idx = 0;
#pragma unroll
    for (int off = 32, n = N; n > 1; off >>= 1, n >>= 1)
        if (lane & off) idx += n / 2;
    return idx;
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Persistent over 128-row groups: block b routes groups b, b + gridDim.x, ...
// (one block per CU). Wr and the bias are staged once per block, and the X
// stream runs on across groups: the loads that would refill the ring after a
// group's last chunks fetch the next group's first chunks instead, so they
// are in flight during the group's epilogue.
template <int EP>
__global__ __launch_bounds__(256, 1) void router_mfma_kernel(RouterParams p) {
    // Staged Wr rows (the MFMA's 32 output columns: rows at or past WROWS
    // enter as zeros) and X buffers per wave. A third buffer (room for it
    // with 16 Wr rows) measured no faster at c3: the stream is bandwidth-bound
    // with two 8 KiB chunks in flight per wave.
    constexpr int WROWS = EP <= 16 ? 16 : 32;
    constexpr int NBUF = 2;
    extern __shared__ uint4 smem_rm[];
    __shared__ int s_cnt[kMaxExperts];
    __shared__ float s_stat[4][kMaxExperts + 1];
    __shared__ float s_fl[4][kMaxExperts + 1];
    __shared__ uint32_t s_flag[4];
    __shared__ float s_bias[kMaxExperts];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int E = p.E, d = p.d, K = p.K;
    const int wpitch = d + 8;  // bf16 elements per staged Wr row
    uint16_t* sw = reinterpret_cast<uint16_t*>(smem_rm);  // [WROWS][wpitch]
    // this wave's NBUF X buffers, [32 rows][128] bf16 each: 16-byte chunk q
    // of row r sits at chunk q ^ (r & 15), so the 32 rows that one fragment
    // read touches spread over the banks
    uint16_t* sx_all = sw + WROWS * wpitch;
    uint16_t* sx = sx_all + wave * NBUF * 32 * 128;
    // flagged rows' logits [kMfmaRouterRows][32] and block-row slots
    float* s_logit = reinterpret_cast<float*>(sx_all + 4 * NBUF * 32 * 128);
    int* s_frow = reinterpret_cast<int*>(s_logit + kMfmaRouterRows * 32);
    if (tid < kMaxExperts) s_cnt[tid] = 0;
    const int nblk = (p.T + kMfmaRouterRows - 1) / kMfmaRouterRows;
    const int rl = lane & 31, hi = lane >> 5;
    const int nch = d / 128;  // d % 128 == 0 (launch check)
    // X loads: load i of a chunk fills rows 4i .. 4i + 3 of the wave's 32
    // (lane -> row 4i + lane / 16, physical chunk lane % 16, which holds the
    // row's logical chunk (lane % 16) ^ (row & 15)): 4 rows x 256 bytes per
    // load instead of the MFMA layout's 32 rows x 32 bytes. Rows past T
    // reload the group's first row; a chunk past the end reloads the last.
    const uint32_t sx0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)sx;
    auto dma_chunk = [&](int g, int c, int buf) {
        const int rb = g * kMfmaRouterRows + wave * 32;
        const int k0 = min(c, nch - 1) * 128;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = 4 * i + (lane >> 4);
            const int rr = rb + r < p.T ? rb + r : g * kMfmaRouterRows;
            dma16_lds(p.X + (int64_t)rr * d + k0 + 8 * ((lane & 15) ^ (r & 15)),
                      sx0 + (uint32_t)(buf * 32 * 128 * 2 + i * 1024));
        }
    };
    // The stream carries across groups only when a group has at least NBUF
    // chunks (its tail loads are then the next group's chunks 0 .. NBUF-1).
    const bool chain = nch >= NBUF;
    int grp = blockIdx.x;
    int qb = 0;  // ring buffer of the group's chunk 0
    // Prologue loads. Where d is a multiple of 512, Wr's rows (1 KiB per
    // load; wave w takes rows w, w + 4, ...) and the bias go straight to LDS
    // ahead of the first group's leading X chunks, so waiting for all but
    // the chunks' loads (the vector-memory counter completes in order) leaves
    // Wr and the bias staged while the chunks are still in flight. A load
    // into registers here would be waited for with the counter at zero,
    // after every chunk. Otherwise the chunks go first and Wr is read through
    // registers, a second round trip overlapping theirs.
    const bool wr_dma = d % 512 == 0;
    const uint32_t sw0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)sw;
    if (wr_dma) {
        for (int n = wave; n < E; n += 4)
            for (int sg = 0; sg < d / 512; ++sg)
                dma16_lds(p.Wr + (int64_t)n * d + sg * 512 + 8 * lane, sw0 + (uint32_t)(n * wpitch * 2 + sg * 1024));
        if (wave == 0 && p.bias != nullptr)  // lanes past E load the last entry (unused)
            dma4_lds(p.bias + min(lane, E - 1),
                     (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)s_bias);
    }
#pragma unroll
    for (int j = 0; j < NBUF; ++j) dma_chunk(grp, j, j);
    if (wr_dma) {
        wait_vmcnt<NBUF * 8>();
    } else {
        if (tid < E && p.bias != nullptr) s_bias[tid] = p.bias[tid];
        // Wr's E rows (rows E .. WROWS-1 zero: their columns are unused).
        // Each block starts at its own offset into the rows, so that the
        // blocks, which all read the same few KiB at kernel start, do not
        // all ask the same L2 lines for them at once.
        const int vpr = d / 8;  // 16-byte vectors per row
        const int nv = E * vpr;
        const int rot = (int)((blockIdx.x * 97u) % (unsigned)nv);
        // 16 loads per thread in flight: one round trip up to E * d = 32 * 1024
        for (int i0 = tid; i0 < nv; i0 += 16 * 256) {
            uint4 v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                int i = min(i0 + u * 256, nv - 1) + rot;
                i = i >= nv ? i - nv : i;
                v[u] = *reinterpret_cast<const uint4*>(p.Wr + (int64_t)i * 8);  // row i / vpr, vector i % vpr
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                if (i0 + u * 256 < nv) {
                    int i = i0 + u * 256 + rot;
                    i = i >= nv ? i - nv : i;
                    const int n = i / vpr, c = i - n * vpr;
                    *reinterpret_cast<uint4*>(sw + n * wpitch + 8 * c) = v[u];
                }
            }
        }
    }
    if (tid < E && p.bias == nullptr) s_bias[tid] = 0.0f;
    for (int i = tid; i < (WROWS - E) * (d / 8); i += 256) {
        const int n = E + i / (d / 8), c = i % (d / 8);
        *reinterpret_cast<uint4*>(sw + n * wpitch + 8 * c) = make_uint4(0, 0, 0, 0);
    }
    __syncthreads();  // Wr and the bias staged
    const uint4 absm = make_uint4(0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu);
    bool leading = true;  // the group's chunks 0 .. NBUF-1 are in flight
    for (; grp < nblk; grp += gridDim.x) {
    const int nxt = grp + (int)gridDim.x;
    if (!leading) {
#pragma unroll
        for (int j = 0; j < NBUF; ++j) dma_chunk(grp, j, j);
        qb = 0;
    }
    const int row_begin = grp * kMfmaRouterRows;
    const int row_end = min(p.T, row_begin + kMfmaRouterRows);
    const int row = row_begin + wave * 32 + rl;
    const bool rvalid = row < row_end;
    f32x16 acc, aab;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = aab[r] = 0.0f;
    // NBUF chunks in flight; every later chunk is requested into the buffer
    // the chunk NBUF before it used, once the wave's reads of that buffer are
    // done (8 loads per chunk: waiting for all but the last (NBUF - 1) * 8
    // leaves the current chunk in LDS)
    for (int c = 0; c < nch; ++c) {
        wait_vmcnt<(NBUF - 1) * 8>();
        const int buf = (qb + c) % NBUF;
        const uint16_t* xb_ = sx + buf * 32 * 128;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int q = (2 * s + hi) ^ (rl & 15);
            const uint4 xa = *reinterpret_cast<const uint4*>(xb_ + rl * 128 + 8 * q);
            uint4 wa = *reinterpret_cast<const uint4*>(sw + (rl & (WROWS - 1)) * wpitch + c * 128 + 16 * s + 8 * hi);
            if (WROWS < 32 && rl >= WROWS) wa = make_uint4(0, 0, 0, 0);
            const uint4 xb = make_uint4(xa.x & absm.x, xa.y & absm.y, xa.z & absm.z, xa.w & absm.w);
            const uint4 wb = make_uint4(wa.x & absm.x, wa.y & absm.y, wa.z & absm.z, wa.w & absm.w);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, wa),
                                                           __builtin_bit_cast(bf16x8, xa), acc, 0, 0, 0);
            aab = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, wb),
                                                           __builtin_bit_cast(bf16x8, xb), aab, 0, 0, 0);
        }
        wait_lgkm0();  // this buffer's reads are done before the next load overwrites it
        const int cn = c + NBUF;
        if (cn < nch) dma_chunk(grp, cn, buf);
        else if (chain && nxt < nblk) dma_chunk(nxt, cn - nch, buf);
        else dma_chunk(grp, nch - 1, buf);  // clamped: keeps the per-chunk load count
    }
    leading = chain && nxt < nblk;
    if (leading) qb = (qb + nch) % NBUF;
    else wait_vmcnt<0>();  // the clamped extra loads, before the buffers are refilled

    // ---- softmax, top K + 1, the separation test (lanes l and l ^ 32 share a
    // row; register r holds expert 8 (r / 4) + 4 (l / 32) + r % 4) ---------
    auto expert_of = [&](int r) { return 8 * (r >> 2) + 4 * hi + (r & 3); };
    float v[16];
    float vmax = -INFINITY, vabs = 0.0f, amax = 0.0f, babs = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int n = expert_of(r);
        const bool ev = n < E;
        // selects, not branches: an expert >= E leaves every maximum as it is
        const float bias = (p.bias != nullptr && ev) ? s_bias[n & (kMaxExperts - 1)] : 0.0f;
        v[r] = p.bias != nullptr ? acc[r] + bias : acc[r];
        vmax = fmaxf(vmax, ev ? v[r] : -INFINITY);
        vabs = fmaxf(vabs, ev ? fabsf(v[r]) : 0.0f);
        amax = fmaxf(amax, ev ? aab[r] : 0.0f);
        babs = fmaxf(babs, fabsf(bias));
    }
    vmax = fmaxf(vmax, xor_lane<32>(vmax));
    vabs = fmaxf(vabs, xor_lane<32>(vabs));
    amax = fmaxf(amax, xor_lane<32>(amax));
    babs = fmaxf(babs, xor_lane<32>(babs));
    float ex[16];
    float se = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        ex[r] = expert_of(r) < E ? __expf(v[r] - vmax) : 0.0f;
        se += ex[r];
    }
    se += xor_lane<32>(se);  // own + partner: both lanes of the row get the same bits
    const float lse = vmax + __logf(se);
    // Top K + 1 by rounds of arg-max over (logit desc, expert asc): per lane
    // the largest candidate (a max tree), then the lowest expert holding it
    // (a min tree over the matching experts; -0 and +0 compare equal, as in a
    // scan with '>' and ties to the lower index), then the partner lane's
    // pick. Experts >= E and picked ones compete as -inf. That equals the
    // exclusion of those experts wherever the row can be clean (every logit
    // of a clean row is finite: an infinite one makes vabs infinite, a NaN
    // makes se NaN, and a round always has a finite candidate); a row that
    // is not clean takes the canonical path below whatever its picks here.
    const int rounds = min(K + 1, E);
    float topv[kMaxTopK + 1];
    int tope[kMaxTopK + 1];
    float cand[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) cand[r] = expert_of(r) < E ? v[r] : -INFINITY;
#pragma unroll
    for (int j = 0; j <= kMaxTopK; ++j) {
        topv[j] = -INFINITY;
        tope[j] = 0;
        if (j < rounds) {
            float tv[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) tv[q] = fmaxf(cand[2 * q], cand[2 * q + 1]);
#pragma unroll
            for (int w = 4; w >= 1; w >>= 1)
#pragma unroll
                for (int q = 0; q < w; ++q) tv[q] = fmaxf(tv[2 * q], tv[2 * q + 1]);
            float bv = tv[0];
            int tn[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) tn[r] = cand[r] == bv ? expert_of(r) : (1 << 20);
#pragma unroll
            for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
                for (int q = 0; q < w; ++q) tn[q] = min(tn[q], tn[q + w]);
            int be = tn[0];
            const float ov = xor_lane<32>(bv);
            const int oe = xor_lane<32>(be);
            if (ov > bv || (ov == bv && oe < be)) {
                bv = ov;
                be = oe;
            }
            topv[j] = bv;
            tope[j] = be;
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (expert_of(r) == be) cand[r] = -INFINITY;
        }
    }
    const float u = 5.9604644775390625e-08f;  // 2^-24
    const float delta =
        (4.0f * (5.0f * (float)d / 64.0f + 24.0f) * 1.001f * amax + 8.0f * (vabs + babs)) * u + 1e-30f;
    bool flag = !(vabs < INFINITY) || !(amax < INFINITY) || !(se > 0.0f);
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j)
        if (j + 1 < rounds && !(topv[j] - topv[j + 1] > 2.0f * delta)) flag = true;
    const bool clean = rvalid && !flag;

    // ---- outputs of the rows that keep the MFMA logits -------------------
    float psum[16];
    float lsum = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) psum[r] = (clean && expert_of(r) < E) ? ex[r] / se : 0.0f;
    if (clean) {
        // register r holds expert 8 (r / 4) + 4 hi + r % 4: four consecutive
        // experts per group of four registers, one 16-byte store each where
        // E is a multiple of 4 (rows then start 16-byte aligned)
        float* lrow = p.logits + (int64_t)row * E;
        float* prow = p.probs + (int64_t)row * E;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int n0 = 8 * q + 4 * hi;
            if ((E & 3) == 0 && n0 < E) {
                *reinterpret_cast<f32x4*>(lrow + n0) = f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
                *reinterpret_cast<f32x4*>(prow + n0) =
                    f32x4{psum[4 * q], psum[4 * q + 1], psum[4 * q + 2], psum[4 * q + 3]};
            } else if ((E & 3) != 0) {
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    if (n0 + t < E) {
                        lrow[n0 + t] = v[4 * q + t];
                        prow[n0 + t] = psum[4 * q + t];
                    }
            }
        }
    }
    if (clean && hi == 0) {
        float zsum = 0.0f, pj[kMaxTopK];
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j) {
            pj[j] = 0.0f;
            if (j < K) {
                pj[j] = __expf(topv[j] - vmax) / se;
                zsum += pj[j];
            }
        }
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j)
            if (j < K) {
                p.idx[(int64_t)row * K + j] = tope[j];
                p.gate[(int64_t)row * K + j] = pj[j] / zsum;
                atomicAdd(&s_cnt[tope[j]], 1);
            }
        p.lse[row] = lse;
        lsum = lse * lse;
    }
    const uint64_t fm = __ballot(rvalid && flag && hi == 0);
    if (lane == 0) s_flag[wave] = (uint32_t)fm;
    // per-wave statistics over the wave's rows, in a fixed order: the xor
    // butterfly (16 .. 1) over the 32 lanes of each half for every register,
    // as a reduce-scatter (each addition pairs the same partial trees as the
    // full butterfly, so the bits are the same): at offset OFF the lane keeps
    // the half of its entries selected by its lane bit OFF; after offset 2
    // lane rl holds register 8 b4 + 4 b3 + 2 b2 + b1 (b_i: bit i of rl), and
    // offset 1 is a plain butterfly step
    {
        auto level = [&](auto off_c, int n) {
            constexpr int OFF = decltype(off_c)::value;
            const bool upper = (lane & OFF) != 0;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                if (t < n) {
                    const float lo = psum[t], hi_ = psum[t + n];
                    const float send = upper ? lo : hi_;
                    const float keep = upper ? hi_ : lo;
                    psum[t] = keep + xor_lane<OFF>(send);
                }
            }
        };
        level(std::integral_constant<int, 16>{}, 8);
        level(std::integral_constant<int, 8>{}, 4);
        level(std::integral_constant<int, 4>{}, 2);
        level(std::integral_constant<int, 2>{}, 1);
        float t = psum[0];
        t += xor_lane<1>(t);
        const int r = ((rl >> 4) & 1) * 8 + ((rl >> 3) & 1) * 4 + ((rl >> 2) & 1) * 2 + ((rl >> 1) & 1);
        const int n = expert_of(r);
        if ((rl & 1) == 0 && n < E) s_stat[wave][n] = t;
    }
    lsum += xor_lane<16>(lsum);
    lsum += xor_lane<8>(lsum);
    lsum += xor_lane<4>(lsum);
    lsum += xor_lane<2>(lsum);
    lsum += xor_lane<1>(lsum);
    if (lane == 0) s_stat[wave][kMaxExperts] = lsum;
    __syncthreads();

    // ---- flagged rows in the canonical order ---------------------------------
    // Logits first: for every flagged row (ascending), wave w computes
    // experts w, w + 4, ... as canonical lane partials over the elements
    // c * 512 + 8 lane + t (fmaf in ascending k) summed by the full xor
    // butterfly (here as one reduce-scatter over the wave's 4 rows x E/4
    // experts), which adds the same partial trees as router_kernel's
    // reduce-scatter. Rows go in batches of 4 with all their X loads in
    // flight together. The logits go to LDS, then softmax / top-k take
    // R = 64 / EP rows per wave pass, lane l holding row l / EP, expert l % EP.
    constexpr int R = 64 / EP;
    constexpr int NCHM = 3;  // 512-element chunks per row: d <= 1536 (router_mfma_fits)
    constexpr int U = EP / 4, V = 4 * U;  // experts per wave, (row, expert) sums per batch
    const uint32_t f0 = s_flag[0], f1 = s_flag[1], f2 = s_flag[2], f3 = s_flag[3];
    const int c0 = __builtin_popcount(f0), c1 = c0 + __builtin_popcount(f1);
    const int c2 = c1 + __builtin_popcount(f2), nflag = c2 + __builtin_popcount(f3);
    float fps = 0.0f, fls = 0.0f;  // per lane: its (row slot, expert)'s sums, folded below
    if (nflag > 0) {
        // the lane's two block-row slots, lane and 64 + lane: flagged, and rank
        // among the block's flagged rows
        const int sh = lane & 31;
        const uint32_t mlo = lane < 32 ? f0 : f1, mhi = lane < 32 ? f2 : f3;
        const uint32_t below = (1u << sh) - 1u;
        const bool flo = (mlo >> sh) & 1u, fhi = (mhi >> sh) & 1u;
        const int rlo = (lane < 32 ? 0 : c0) + __builtin_popcount(mlo & below);
        const int rhi = (lane < 32 ? c1 : c2) + __builtin_popcount(mhi & below);
        auto nth_flagged = [&](int i) -> int {  // block-row slot of flagged row i < nflag
            const uint64_t bl = __ballot(flo && rlo == i);
            if (bl != 0) return __builtin_ctzll(bl);
            return 64 + __builtin_ctzll(__ballot(fhi && rhi == i));
        };
        const int nch = (d + 511) / 512;
        // the entry this lane's sum ends on, and whether it writes it
        const int ent = rs_sum_entry<V>(lane);
        const bool writer = (lane & (64 / V - 1)) == 0;
        for (int i0 = 0; i0 < nflag; i0 += 4) {
            int frow[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) frow[r] = i0 + r < nflag ? row_begin + nth_flagged(i0 + r) : -1;
            if (wave == 0 && lane < 4 && i0 + lane < nflag) {
                int fr = frow[0];
#pragma unroll
                for (int r = 1; r < 4; ++r)
                    if (lane == r) fr = frow[r];
                s_frow[i0 + lane] = fr;
            }
            uint4 xv[4][NCHM];
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int c = 0; c < NCHM; ++c) {
                    const int k = c * 512 + 8 * lane;
                    const bool ok = frow[r] >= 0 && c < nch && k < d;  // clamped: no load under a branch
                    xv[r][c] = *reinterpret_cast<const uint4*>(p.X + (int64_t)(ok ? frow[r] : row_begin) * d +
                                                               (ok ? k : 0));
                }
            float a[V];  // entry r * U + u: row i0 + r, expert wave + 4u
#pragma unroll
            for (int i = 0; i < V; ++i) a[i] = 0.0f;
#pragma unroll
            for (int c = 0; c < NCHM; ++c) {
                if (c < nch) {
                    const int k = c * 512 + 8 * lane;
                    const bool ok = k < d;  // a lane past d keeps its partials
                    float xf[4][8];
#pragma unroll
                    for (int r = 0; r < 4; ++r) unpack8(xv[r][c], xf[r]);
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const int e = wave + 4 * u;
                        if (e < E) {
                            float wf[8];
                            unpack8(*reinterpret_cast<const uint4*>(sw + e * wpitch + (ok ? k : 0)), wf);
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                float t = a[r * U + u];
#pragma unroll
                                for (int q = 0; q < 8; ++q) t = __builtin_fmaf(xf[r][q], wf[q], t);
                                a[r * U + u] = ok ? t : a[r * U + u];
                            }
                        }
                    }
                }
            }
            rs_sum_level<32, V>(a, lane);
            const int rr = ent / U, e = wave + 4 * (ent % U);
            if (writer && i0 + rr < nflag && e < E)
                s_logit[(i0 + rr) * E + e] = p.bias != nullptr ? a[0] + s_bias[e] : a[0];
        }
        __syncthreads();
        const int e_mine = lane % EP, r_mine = lane / EP;
        const bool e_valid = e_mine < E;
        for (int g0 = wave * R; g0 < nflag; g0 += 4 * R) {
            const int i = g0 + r_mine;
            const bool rv = i < nflag;
            const float logit = rv && e_valid ? s_logit[i * E + e_mine] : 0.0f;
            const RowPick pk = softmax_topk<EP>(logit, e_valid, e_mine, K);
            if (rv) {
                const int frw = s_frow[i];
                if (e_valid) {
                    p.logits[(int64_t)frw * E + e_mine] = logit;
                    p.probs[(int64_t)frw * E + e_mine] = pk.prob;
                    fps += pk.prob;
                    if (pk.sel) atomicAdd(&s_cnt[e_mine], 1);
                }
                if (e_mine < K) {
                    p.idx[(int64_t)frw * K + e_mine] = pk.idx;
                    p.gate[(int64_t)frw * K + e_mine] = pk.gate;
                }
                if (e_mine == 0) {
                    p.lse[frw] = pk.lse;
                    fls += pk.lse * pk.lse;
                }
            }
        }
    }
    // fold the row slots: lane e < EP holds expert e's sum, lane 0 the lse^2 sum
    if constexpr (EP <= 32) { fps += xor_lane<32>(fps); fls += xor_lane<32>(fls); }
    if constexpr (EP <= 16) { fps += xor_lane<16>(fps); fls += xor_lane<16>(fls); }
    if constexpr (EP <= 8) { fps += xor_lane<8>(fps); fls += xor_lane<8>(fls); }
    if (lane < E) s_fl[wave][lane] = fps;
    if (lane == 0) s_fl[wave][kMaxExperts] = fls;
    __syncthreads();
    const int blk = grp;
    if (tid <= E) {
        const int col = tid < E ? tid : kMaxExperts;
        float t = s_stat[0][col];
        t += s_stat[1][col];
        t += s_stat[2][col];
        t += s_stat[3][col];
        t += s_fl[0][col];
        t += s_fl[1][col];
        t += s_fl[2][col];
        t += s_fl[3][col];
        p.blkstat[(int64_t)blk * (E + 1) + tid] = t;
        if (tid < E) {
            p.blkcnt[(int64_t)blk * E + tid] = s_cnt[tid];
            s_cnt[tid] = 0;  // for the next group (after the barrier below)
        }
    }
    // the next group rewrites the statistics, flags and counts read above
    __syncthreads();
    }
}

// Dynamic LDS of router_mfma_kernel: staged Wr rows, the X buffers, the
// flagged rows' logits and slots.
static size_t router_mfma_lds(int d, int E) {
    const int ep = router_ep(E);
    const size_t wrows = ep <= 16 ? 16 : 32, nbuf = 2;
    return wrows * (d + 8) * 2 + 4 * nbuf * 32 * 128 * 2 + (size_t)kMfmaRouterRows * 32 * 4 + kMfmaRouterRows * 4;
}

bool router_mfma_fits(int T, int E, int K, int d) {
    return E >= 2 && E <= 32 && K <= E && K <= kMaxTopK && d % 128 == 0 && d >= 128 && d <= 3 * 512 &&
           router_mfma_lds(d, E) + 4096 <= 160 * 1024 && (T + kMfmaRouterRows - 1) / kMfmaRouterRows >= cu_count();
}

hipError_t launch_router_mfma(const RouterParams& p, int nblk, hipStream_t s) {
    if (p.rows_per_block != kMfmaRouterRows || p.ln_H != nullptr || !router_mfma_fits(nblk * kMfmaRouterRows, p.E, p.K, p.d) ||
        nblk != (p.T + kMfmaRouterRows - 1) / kMfmaRouterRows)
        return hipErrorInvalidValue;
    const size_t lds = router_mfma_lds(p.d, p.E);
    // one block per CU (its LDS), each walking the 128-row groups b, b + grid, ...
    const int grid = min(nblk, cu_count());
    switch (router_ep(p.E)) {
        case 8: router_mfma_kernel<8><<<grid, 256, lds, s>>>(p); break;
        case 16: router_mfma_kernel<16><<<grid, 256, lds, s>>>(p); break;
        case 32: router_mfma_kernel<32><<<grid, 256, lds, s>>>(p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// LayerNorm chunks of the fused router: 512-element chunks rounded up to 1, 2
// or 4; a wave holds R = 64 / EP rows of them in registers (R * NCH <= 16;
// with 64 expert lanes, whose 64 partials per lane leave less room, NCH <= 2).
static int router_ln_chunks(int E, int d) {
    const int nch = (d + 511) / 512;
    const int c = nch <= 1 ? 1 : nch <= 2 ? 2 : nch <= 4 ? 4 : 0;
    const bool fits = c > 0 && router_rows_per_wave(E) * c <= 16 && (router_ep(E) < 64 || c <= 2);
    return fits ? c : 0;
}
bool router_ln_fits(int E, int d) { return router_ln_chunks(E, d) > 0; }

hipError_t launch_router(const RouterParams& p, int nblk, hipStream_t s) {
    const bool wlds = router_wr_in_lds(p.E, p.d);
    const size_t lds = wlds ? (size_t)p.E * p.d * 2 : 0;
    const int ep = router_ep(p.E);
    const int nch = p.ln_H != nullptr ? router_ln_chunks(p.E, p.d) : 0;
    if (p.ln_H != nullptr && nch == 0) return hipErrorInvalidValue;
    dim3 grid(nblk), block(64 * kRouterWaves);
#define TMT_ROUTER_NCH(EP_, NCH_)                                                               \
    if (wlds) router_kernel<EP_, true, kRouterWaves, NCH_><<<grid, block, lds, s>>>(p);        \
    else router_kernel<EP_, false, kRouterWaves, NCH_><<<grid, block, 0, s>>>(p);
#define TMT_ROUTER(EP_)                              \
    case EP_:                                        \
        if (nch == 0) { TMT_ROUTER_NCH(EP_, 0) }     \
        else if (nch == 1) { TMT_ROUTER_NCH(EP_, 1) } \
        else if (nch == 2) { TMT_ROUTER_NCH(EP_, 2) } \
        else if constexpr (EP_ > 8 && EP_ < 64) { TMT_ROUTER_NCH(EP_, 4) } \
        break;
    switch (ep) {
        TMT_ROUTER(8)
        TMT_ROUTER(16)
        TMT_ROUTER(32)
        TMT_ROUTER(64)
        default: return hipErrorInvalidValue;
    }
#undef TMT_ROUTER
#undef TMT_ROUTER_NCH
    return hipGetLastError();
}

// From the per-expert totals s_cnt and the summed block statistics s_fsum
// (E probability sums, then the lse^2 sum): the exclusive offsets into s_off
// and, with `stats`, the switch aux (moe.cu:456-465) and z-loss mean
// (moe.cu:268-278). One thread.
__device__ __forceinline__ void scan_offsets_stats(const ScanParams& p, const int* s_cnt, const float* s_fsum,
                                                   int* s_off, bool stats) {
    const int E = p.E;
    int run = 0;
    for (int e = 0; e < E; ++e) {
        s_off[e] = run;
        run += s_cnt[e];
    }
    s_off[E] = run;
    if (!stats) return;
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
// Expert e's count (in counts and stats) and its place in the descending-
// count order (ties to the lower index).
__device__ __forceinline__ void scan_write_expert(const ScanParams& p, const int* s_cnt, int e) {
    p.counts[e] = s_cnt[e];
    reinterpret_cast<int32_t*>(p.stats + 2)[e] = s_cnt[e];
    int rank = 0;
    for (int q = 0; q < p.E; ++q) rank += (s_cnt[q] > s_cnt[e]) || (s_cnt[q] == s_cnt[e] && q < e);
    p.order[rank] = e;
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

    // 1) per (segment, expert) sums of the block histograms (no more
    // segments than blocks: the serial scans of step 2 walk every segment)
    const int S = max(1, min(1024 / E, nblk));
    const int chunk = (nblk + S - 1) / S;
    // (Loads in batches of 8 at clamped addresses, added in ascending order:
    // one memory round trip per batch instead of one per block.)
    if (tid < S * E) {
        const int e = tid % E, seg = tid / E;
        const int b0 = seg * chunk, b1 = min(nblk, b0 + chunk);
        int sum = 0;
        for (int b = b0; b < b1; b += 8) {
            int v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = p.blkcnt[(int64_t)min(b + u, b1 - 1) * E + e];
#pragma unroll
            for (int u = 0; u < 8; ++u) sum += b + u < b1 ? v[u] : 0;
        }
        s_seg[seg * E + e] = sum;
    }
    // 1b) per (segment, statistic) sums of the block statistics
    const int E1 = E + 1;
    const int S2 = max(1, min(1024 / E1, nblk));
    const int chunk2 = (nblk + S2 - 1) / S2;
    if (tid < S2 * E1) {
        const int q = tid % E1, seg = tid / E1;
        const int b0 = seg * chunk2, b1 = min(nblk, b0 + chunk2);
        float sum = 0.0f;
        for (int b = b0; b < b1; b += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = p.blkstat[(int64_t)min(b + u, b1 - 1) * E1 + q];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (b + u < b1) sum += v[u];
        }
        s_fseg[seg * E1 + q] = sum;
    }
    __syncthreads();
    // 2) exclusive scan over segments, per expert
    if (tid < E) {
        int run = 0;
        for (int seg0 = 0; seg0 < S; seg0 += 8) {
            int c[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) c[u] = s_seg[min(seg0 + u, S - 1) * E + tid];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (seg0 + u < S) {
                    s_seg[(seg0 + u) * E + tid] = run;
                    run += c[u];
                }
            }
        }
        s_cnt[tid] = run;
    }
    if (tid < E1) {
        float run = 0.0f;
        for (int seg0 = 0; seg0 < S2; seg0 += 8) {
            float c[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) c[u] = s_fseg[min(seg0 + u, S2 - 1) * E1 + tid];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (seg0 + u < S2) run += c[u];
        }
        s_fsum[tid] = run;
    }
    __syncthreads();
    if (tid == 0) scan_offsets_stats(p, s_cnt, s_fsum, s_off, true);
    __syncthreads();
    if (tid <= E) p.offsets[tid] = s_off[tid];
    if (tid < E) scan_write_expert(p, s_cnt, tid);
    // 3) per-block bases
    if (tid < S * E) {
        const int e = tid % E, seg = tid / E;
        const int b0 = seg * chunk, b1 = min(nblk, b0 + chunk);
        int run = s_off[e] + s_seg[seg * E + e];
        for (int b = b0; b < b1; b += 8) {
            int v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = p.blkcnt[(int64_t)min(b + u, b1 - 1) * E + e];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (b + u < b1) {
                    p.blkbase[(int64_t)(b + u) * E + e] = run;
                    run += v[u];
                }
            }
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

// The permutation with the scan folded in, for grids of at most
// kFusedScanBlocks router blocks: every block adds the block histograms
// itself (the totals, and the counts of the blocks before it, in ascending
// block order) to find its own bases, and block 0 writes the counts,
// offsets, order and statistics (block statistics added in ascending block
// order). One launch fewer where the scan's single workgroup was mostly
// launch latency. Slots are the same as scan_kernel + permute_kernel give.
__global__ __launch_bounds__(kThreads) void permute_scan_kernel(PermuteParams p, ScanParams sp) {
    __shared__ int s_g[kMaxGroups][kMaxExperts];
    __shared__ int s_tot[kMaxExperts];
    __shared__ int s_base[kMaxExperts];
    __shared__ int s_off[kMaxExperts + 1];
    __shared__ float s_fsum[kMaxExperts + 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = p.K, E = p.E, nblk = sp.nblk, b = blockIdx.x;
    if (tid < E) {
        int tot = 0, before = 0;
        for (int b0 = 0; b0 < nblk; b0 += 8) {
            int v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = sp.blkcnt[(int64_t)min(b0 + u, nblk - 1) * E + tid];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int c = b0 + u < nblk ? v[u] : 0;
                tot += c;
                before += b0 + u < b ? c : 0;
            }
        }
        s_tot[tid] = tot;
        s_base[tid] = before;
    } else if (b == 0 && tid >= 64 && tid - 64 <= E) {
        const int q = tid - 64;
        float run = 0.0f;
        for (int b0 = 0; b0 < nblk; b0 += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = sp.blkstat[(int64_t)min(b0 + u, nblk - 1) * (E + 1) + q];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (b0 + u < nblk) run += v[u];
        }
        s_fsum[q] = run;
    }
    __syncthreads();
    if (tid == 0) scan_offsets_stats(sp, s_tot, s_fsum, s_off, b == 0);
    __syncthreads();
    if (tid < E) {
        s_base[tid] += s_off[tid];
        if (b == 0) scan_write_expert(sp, s_tot, tid);
    }
    if (b == 0 && tid <= E) sp.offsets[tid] = s_off[tid];
    // the permutation (permute_kernel with the block bases from s_base)
    const int RG = 64 / K;
    const int pairs = RG * K;
    const int row_begin = b * p.rows_per_block;
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
        int run = s_base[tid];
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

hipError_t launch_permute_scan(const PermuteParams& p, const ScanParams& sp, int nblk, hipStream_t s) {
    const int RG = 64 / p.K;
    if ((p.rows_per_block + RG - 1) / RG > kMaxGroups || nblk < 1 || nblk > kFusedScanBlocks || p.E > kMaxExperts)
        return hipErrorInvalidValue;
    permute_scan_kernel<<<nblk, kThreads, 0, s>>>(p, sp);
    return hipGetLastError();
}

hipError_t launch_permute(const PermuteParams& p, int nblk, hipStream_t s) {
    const int RG = 64 / p.K;
    if ((p.rows_per_block + RG - 1) / RG > kMaxGroups) return hipErrorInvalidValue;
    permute_kernel<<<nblk, kThreads, 0, s>>>(p);
    return hipGetLastError();
}

// T <= kSmallRouteTokens (decode): router, counts, offsets, statistics,
// expert order and the stable permutation in one launch instead of router +
// scan + permute. One 4-wave block per token row:
//  1. the row's E logits: wave w computes experts w, w + 4, ..., each as the
//     canonical lane partials and the full xor butterfly (32 .. 1), which adds
//     the same partial trees as router_kernel's reduce-scatter (bit-identical);
//  2. softmax / top-k / gates of the row on EP lanes (router_kernel's code);
//     a single token's dispatch follows from wave 0's registers directly;
//  3. with more than one row, the last block to finish (an atomic ticket,
//     device-scope fences on both sides) reads every row's picks back and
//     computes counts, offsets, aux / z, the expert order and the stable
//     permutation, and re-arms the ticket.
// Decode steps are latency-bound and one wave issues one instruction every
// few cycles, so the serial parts are short and spread over the waves, and
// the last block issues its stores after its last barrier (a barrier waits
// for the block's outstanding global stores).
constexpr int kSmallGroups = 8;  // ceil(T / floor(64 / K)) for T <= 64, K <= 8

template <int EP>
__global__ __launch_bounds__(kThreads) void route_small_kernel(RouterParams p, ScanParams sp,
                                                               PermuteParams pp, int* ticket) {
    __shared__ float s_logit[kMaxExperts];
    __shared__ float s_sum[kMaxExperts + 1];
    __shared__ int s_cnt[kMaxExperts];
    __shared__ int s_idx[kSmallRouteTokens * kMaxTopK];
    __shared__ float s_prob[kSmallRouteTokens * kMaxExperts];
    __shared__ float s_lse[kSmallRouteTokens];
    __shared__ int s_off[kMaxExperts + 1];
    __shared__ int s_g[kSmallGroups][kMaxExperts];
    __shared__ int s_last;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = p.E, K = p.K, T = p.T;
    const int row = blockIdx.x;
    const bool single = gridDim.x == 1;

    // 1. logits of this row (one memory round trip: every load of a pass is
    // in flight together)
    token_logits(p, row, s_logit, wave, 4, lane);
    __syncthreads();

    // 2. softmax, top-k, gates on EP lanes of wave 0; one token finishes
    // here, several publish their row for the last block.
    if (wave == 0) {
        const int e = lane % EP;
        const bool ev = lane < EP && e < E;
        const float logit = ev ? s_logit[e] : 0.0f;
        const RowPick pk = softmax_topk<EP>(logit, ev, e, K);
        if (single) {
            one_token_dispatch<EP>(p, sp, pp, logit, ev, pk, lane);
        } else if (lane < EP) {
            if (ev) {
                p.logits[(int64_t)row * E + e] = logit;
                p.probs[(int64_t)row * E + e] = pk.prob;
            }
            if (e < K) {
                p.idx[(int64_t)row * K + e] = pk.idx;
                p.gate[(int64_t)row * K + e] = pk.gate;
            }
            if (e == 0) p.lse[row] = pk.lse;
        }
    }
    if (single || ticket == nullptr) return;

    // 3. the last block finishes the dispatch (every row read back in one batch)
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = atomicAdd(ticket, 1) == T - 1;
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    {
        // All of a thread's loads are issued before any LDS store.
        const int ni = T * K, np = T * E, n = ni + np + T;
        const uint32_t* gidx = reinterpret_cast<const uint32_t*>(p.idx);
        const uint32_t* gprob = reinterpret_cast<const uint32_t*>(p.probs);
        const uint32_t* glse = reinterpret_cast<const uint32_t*>(p.lse);
        for (int base = tid; base < n; base += 8 * kThreads) {
            uint32_t v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int i = min(base + u * kThreads, n - 1);
                v[u] = i < ni ? gidx[i] : (i < ni + np ? gprob[i - ni] : glse[i - ni - np]);
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int i = base + u * kThreads;
                if (i >= n) break;
                if (i < ni) s_idx[i] = (int)v[u];
                else if (i < ni + np) s_prob[i - ni] = __uint_as_float(v[u]);
                else s_lse[i - ni - np] = __uint_as_float(v[u]);
            }
        }
    }
    __syncthreads();

    // Per-expert probability sums over the rows in order (wave 3), the sum
    // of lse^2 (wave 2) and the per-group pick counts of the stable
    // permutation (groups of floor(64/K) tokens, a ballot per expert, waves
    // g < G). Loops over experts and groups run to the compile-time bounds
    // EP and kSmallGroups, so their LDS reads are issued together.
    if (wave == 3 && lane < E) {
        float sum = 0.0f;
        for (int r0 = 0; r0 < T; r0 += 8) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = s_prob[min(r0 + i, T - 1) * E + lane];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (r0 + i < T) sum += v[i];
        }
        s_sum[lane] = sum;
    } else if (wave == 2 && lane == 0) {
        float sum = 0.0f;
        for (int r0 = 0; r0 < T; r0 += 8) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float l = s_lse[min(r0 + i, T - 1)];
                v[i] = l * l;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (r0 + i < T) sum += v[i];
        }
        s_sum[E] = sum;
    }
    const int RG = 64 / K, pairs = RG * K;
    const int G = (T + RG - 1) / RG;
    const int rr = lane / K, j = lane % K;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int g = wave; g < G; g += 4) {
        const int r = g * RG + rr;
        const bool valid = lane < pairs && r < T;
        const int e = valid ? s_idx[r * K + j] : -1;
#pragma unroll
        for (int ee = 0; ee < EP; ++ee) {
            const uint64_t m = __ballot(e == ee);
            if (lane == ee) s_g[g][ee] = __popcll(m);
        }
    }
    __syncthreads();

    // Counts (the groups' counts added), offsets (an exclusive scan over the
    // expert lanes) and the group bases of each expert's segment, on wave 0.
    if (wave == 0) {
        int c[kSmallGroups], cnt = 0;
#pragma unroll
        for (int g = 0; g < kSmallGroups; ++g) {
            c[g] = (g < G && lane < E) ? s_g[g][lane] : 0;
            cnt += c[g];
        }
        int incl = cnt;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(incl, o, 64);
            if (lane >= o) incl += t;
        }
        int run = incl - cnt;
        if (lane < E) {
            s_cnt[lane] = cnt;
            s_off[lane] = run;
#pragma unroll
            for (int g = 0; g < kSmallGroups; ++g) {
                if (g < G) s_g[g][lane] = run;
                run += c[g];
            }
        }
        if (lane == 0) s_off[E] = T * K;
    }
    __syncthreads();

    // Everything that is stored is computed first: a register that still
    // feeds an outstanding store cannot be overwritten without a wait.
    int pos[2], prow[2];
    bool pvalid[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {  // G <= kSmallGroups = 8 groups over 4 waves
        const int g = wave + 4 * q;
        const int r = g * RG + rr;
        pvalid[q] = g < G && lane < pairs && r < T;
        pos[q] = 0;
        prow[q] = r;
        if (g >= G) continue;  // uniform
        const int e = pvalid[q] ? s_idx[r * K + j] : -1;
        int rank = 0;
#pragma unroll
        for (int ee = 0; ee < EP; ++ee) {
            const uint64_t m = __ballot(e == ee);
            if (e == ee) rank = __popcll(m & lt_mask);
        }
        if (pvalid[q]) pos[q] = s_g[g][e] + rank;
    }
    // Expert order on wave 1, aux / z on wave 2.
    int ord = 0, cnt = 0, off = 0;
    if (tid <= E) off = s_off[tid];
    const bool order_lane = wave == 1 && lane < E;
    if (order_lane) {
        cnt = s_cnt[lane];
#pragma unroll
        for (int e = 0; e < EP; ++e) {
            const int ce = s_cnt[e];
            ord += e < E && ((ce > cnt) || (ce == cnt && e < lane));
        }
    }
    float aux = 0.0f, zl = 0.0f;
    const bool stat_lane = wave == 2 && lane == 0;
    if (stat_lane) {
        // Switch aux (moe.cu:456-465) and z-loss mean (moe.cu:268-278).
        const float inv_t = 1.0f / (float)T;
        const float inv_tk = 1.0f / ((float)T * (float)K);
        float fs[EP], fc[EP];
#pragma unroll
        for (int e = 0; e < EP; ++e) {
            fs[e] = s_sum[min(e, E - 1)];
            fc[e] = (float)s_cnt[e];
        }
#pragma unroll
        for (int e = 0; e < EP; ++e)
            if (e < E) aux += (fs[e] * inv_t) * (fc[e] * inv_tk);
        aux *= (float)E;
        zl = s_sum[E] * inv_t;
    }
    // Stores only from here on.
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        if (pvalid[q]) {
            pp.perm[pos[q]] = prow[q];
            pp.slot_of[(int64_t)prow[q] * K + j] = pos[q];
        }
    }
    if (tid <= E) sp.offsets[tid] = off;
    if (order_lane) {
        sp.counts[lane] = cnt;
        reinterpret_cast<int32_t*>(sp.stats + 2)[lane] = cnt;
        sp.order[ord] = lane;
    }
    if (stat_lane) {
        sp.stats[0] = aux;
        sp.stats[1] = zl;
        *ticket = 0;  // re-armed for the next call (stream order keeps calls apart)
    }
}

hipError_t launch_route_small(const RouterParams& p, const ScanParams& sp, const PermuteParams& pp,
                              int* ticket, hipStream_t s) {
    if (p.T < 1 || p.T > kSmallRouteTokens || p.K > kMaxTopK) return hipErrorInvalidValue;
    if ((p.T + 64 / p.K - 1) / (64 / p.K) > kSmallGroups) return hipErrorInvalidValue;
    dim3 grid(p.T), block(kThreads);
    switch (router_ep(p.E)) {
        case 8: route_small_kernel<8><<<grid, block, 0, s>>>(p, sp, pp, ticket); break;
        case 16: route_small_kernel<16><<<grid, block, 0, s>>>(p, sp, pp, ticket); break;
        case 32: route_small_kernel<32><<<grid, block, 0, s>>>(p, sp, pp, ticket); break;
        case 64: route_small_kernel<64><<<grid, block, 0, s>>>(p, sp, pp, ticket); break;
        default: return hipErrorInvalidValue;
    }
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
