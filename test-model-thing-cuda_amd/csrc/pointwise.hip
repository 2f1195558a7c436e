// pointwise.hip -- HBM-bound MoE kernels around the grouped GEMMs.
//
//   combine      Y_r = beta*Y_r + sum_j gate_rj * O[slot(r,j)]
//                (reference combine_kernel, tmt-cuda/src/moe.cu:142-158)
//   combine_bwd  s_rj = dY_r . O[slot], dO[slot] = gate_rj * dY_r, and the
//                router gradient of row r through renorm + softmax + aux + z
//                (moe.cu:160-234, fused; one wave per token row); also copies
//                X_r to Xg[slot] (the reference's gather recompute, moe.cu:497-502)
//   router_dw    dWr = dlogits^T X with a fixed-order two-pass reduction
//                (moe.cu:521; no atomics)
//   scatter      dX_r = sum_j dXg[slot(r,j)] + dlogits_r . Wr  (moe.cu:236-249
//                and the router input gradient moe.cu:522-531, fused)
// Rows are processed by one 64-lane wave with 16-byte vectors; every sum runs
// in a fixed order, so results are run-to-run deterministic.
#include <algorithm>

#include "device_util.hpp"
#include "dispatch.hpp"
#include "moe_internal.hpp"

namespace tmt {
namespace {

// self_dispatch: the grid's extra (last) workgroup writes the dispatch
// tables from the pick table; true for that workgroup.
__device__ __forceinline__ bool combine_tables_block(const CombineParams& p, int lane) {
    if ((int)blockIdx.x != (int)gridDim.x - 1) return false;
    if (threadIdx.x < 64) {
        int ent[kPickGroups];
        load_pick_table(p.idx, p.T * p.K, lane, ent);
        write_dispatch(p.tables, ent, lane);
    }
    return true;
}

// Slots and gates of row r's K picks: from slot_of, or (self_dispatch) from
// the pick table.
template <int K>
__device__ __forceinline__ void row_picks(const CombineParams& p, int r, int lane, int64_t (&pos)[K], float (&g)[K]) {
    if (p.self_dispatch) {
        int ent[kPickGroups];
        load_pick_table(p.idx, p.T * K, lane, ent);
        int e[K];
#pragma unroll
        for (int j = 0; j < K; ++j) {
            e[j] = p.idx[(int64_t)r * K + j];
            g[j] = p.gate[(int64_t)r * K + j];
        }
#pragma unroll
        for (int j = 0; j < K; ++j) pos[j] = pick_slot(ent, p.T * K, e[j], r * K + j, lane);
    } else {
#pragma unroll
        for (int j = 0; j < K; ++j) {
            pos[j] = p.slot_of[(int64_t)r * K + j];
            g[j] = p.gate[(int64_t)r * K + j];
        }
    }
}

// K is a template argument so that every load of a pass is issued
// unconditionally, in one batch: with a runtime K the compiler places the
// loads under per-pick branches and waits between them.
template <bool SILU, int K>
__global__ __launch_bounds__(kThreads) void combine_kernel(CombineParams p) {
    const int lane = threadIdx.x & 63;
    if (p.self_dispatch && combine_tables_block(p, lane)) return;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= p.T) return;
    const int d = p.d;
    int64_t pos[K];
    float g[K];
    row_picks<K>(p, r, lane, pos, g);
    const bool resid = p.beta != 0.0f;
    // Two 512-column chunks per pass with all their loads in flight together
    // (a decode row waits for one round trip after the slot table, not one
    // per chunk). A lane whose second chunk lies past d reloads its first
    // and stores it once.
    for (int cb = lane * 8; cb < d; cb += 1024) {
        const bool two = cb + 512 < d;
        const int cc[2] = {cb, two ? cb + 512 : cb};
        uint4 yv[2], ov[2][K];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            yv[h] = resid ? *reinterpret_cast<const uint4*>(p.Y + (int64_t)r * d + cc[h]) : make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < K; ++j) ov[h][j] = *reinterpret_cast<const uint4*>(p.O + (int64_t)pos[j] * d + cc[h]);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float acc[8];
            if (resid) {
                unpack8(yv[h], acc);
#pragma unroll
                for (int t = 0; t < 8; ++t) acc[t] *= p.beta;
            } else {
#pragma unroll
                for (int t = 0; t < 8; ++t) acc[t] = 0.0f;
            }
#pragma unroll
            for (int j = 0; j < K; ++j) {
                float o[8];
                unpack8(ov[h][j], o);
#pragma unroll
                for (int t = 0; t < 8; ++t) acc[t] += g[j] * (SILU ? silu_fast(o[t]) : o[t]);
            }
            if (h == 0 || two) *reinterpret_cast<uint4*>(p.Y + (int64_t)r * d + cc[h]) = pack8(acc);
        }
    }
}

// Decode GEMM_DOWN split in K halves: O[slot] = bf16(part[0][slot] +
// part[1][slot]) is formed (and stored for the backward), then combined as in
// combine_kernel<false, K> with the rounded values. One 512-column chunk per
// pass, every load of the pass issued first.
template <int K>
__global__ __launch_bounds__(kThreads) void combine_part_kernel(CombineParams p) {
    const int lane = threadIdx.x & 63;
    if (p.self_dispatch && combine_tables_block(p, lane)) return;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= p.T) return;
    const int d = p.d;
    const int64_t half = (int64_t)p.slots * d;
    int64_t pos[K];
    float g[K];
    row_picks<K>(p, r, lane, pos, g);
    const bool resid = p.beta != 0.0f;
    for (int c0 = lane * 8; c0 < d; c0 += 512) {
        const uint4 yv = resid ? *reinterpret_cast<const uint4*>(p.Y + (int64_t)r * d + c0) : make_uint4(0, 0, 0, 0);
        f32x4 a[K][4];
#pragma unroll
        for (int j = 0; j < K; ++j) {
            const float* q = p.part + pos[j] * d + c0;
            a[j][0] = *reinterpret_cast<const f32x4*>(q);
            a[j][1] = *reinterpret_cast<const f32x4*>(q + 4);
            a[j][2] = *reinterpret_cast<const f32x4*>(q + half);
            a[j][3] = *reinterpret_cast<const f32x4*>(q + half + 4);
        }
        float acc[8];
        if (resid) {
            unpack8(yv, acc);
#pragma unroll
            for (int t = 0; t < 8; ++t) acc[t] *= p.beta;
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) acc[t] = 0.0f;
        }
#pragma unroll
        for (int j = 0; j < K; ++j) {
            float s8[8], o[8];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                s8[t] = a[j][0][t] + a[j][2][t];
                s8[t + 4] = a[j][1][t] + a[j][3][t];
            }
            const uint4 ob = pack8(s8);
            *reinterpret_cast<uint4*>(p.O_out + pos[j] * d + c0) = ob;
            unpack8(ob, o);
#pragma unroll
            for (int t = 0; t < 8; ++t) acc[t] += g[j] * o[t];
        }
        *reinterpret_cast<uint4*>(p.Y + (int64_t)r * d + c0) = pack8(acc);
    }
}

// One pass over the row's 512-column chunks: each chunk of dY and X is loaded
// once for all K picks (re-reading them per pick missed in L2 behind the
// dO / Xg stores), with the K gathered O chunks in flight together. Each
// pick's partial dot product still runs over the chunks in ascending order.
template <bool SILU, int K>
__global__ __launch_bounds__(kThreads) void combine_bwd_kernel(CombineBwdParams p) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= p.T) return;
    const int d = p.d, E = p.E;
    int64_t pos[K];
    float gj[K], part[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
        pos[j] = p.slot_of[(int64_t)r * K + j];
        gj[j] = p.gate[(int64_t)r * K + j];
        part[j] = 0.0f;
    }
    for (int c0 = lane * 8; c0 < d; c0 += 512) {
        const uint4 dyv = *reinterpret_cast<const uint4*>(p.dY + (int64_t)r * d + c0);
        const uint4 xv = *reinterpret_cast<const uint4*>(p.X + (int64_t)r * d + c0);
        uint4 ov[K];
#pragma unroll
        for (int j = 0; j < K; ++j) ov[j] = *reinterpret_cast<const uint4*>(p.O + pos[j] * d + c0);
        float dy[8];
        unpack8(dyv, dy);
#pragma unroll
        for (int j = 0; j < K; ++j) {
            float o[8], out[8];
            unpack8(ov[j], o);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                if (SILU) {
                    // Reference experts: gradient through the SiLU applied in
                    // combine (combine_bwd_kernel, moe.cu:162-176).
                    part[j] += dy[t] * silu_fast(o[t]);
                    out[t] = gj[j] * dy[t] * dsilu_fast(o[t]);
                } else {
                    part[j] += dy[t] * o[t];
                    out[t] = gj[j] * dy[t];
                }
            }
            *reinterpret_cast<uint4*>(p.dO + pos[j] * d + c0) = pack8(out);
            *reinterpret_cast<uint4*>(p.Xg + pos[j] * d + c0) = xv;
        }
    }
    float s[K];
#pragma unroll
    for (int j = 0; j < K; ++j) s[j] = wave_sum(part[j]);
    if (E <= 1) return;

    // Router backward for row r, lane e (router_bwd_kernel, moe.cu:199-234).
    const int e = lane;
    const bool ev = e < E;
    const float pe = ev ? p.probs[(int64_t)r * E + e] : 0.0f;
    float Z = 0.0f, sp = 0.0f, g = 0.0f;
    int ej[K];
#pragma unroll
    for (int j = 0; j < K; ++j) ej[j] = p.idx[(int64_t)r * K + j];
#pragma unroll
    for (int j = 0; j < K; ++j) {
        const float pj = p.probs[(int64_t)r * E + ej[j]];
        Z += pj;
        sp += s[j] * pj;
    }
    const float Z2 = Z * Z + 1e-12f;
#pragma unroll
    for (int j = 0; j < K; ++j) {
        if (ej[j] == e) g = (s[j] * Z - sp) / Z2;
    }
    const float inv_tk = 1.0f / ((float)p.T * (float)K);
    const float frac = ev ? (float)p.counts[e] * inv_tk : 0.0f;
    const float acc = wave_sum(g * pe);
    const float expected = wave_sum(pe * frac);
    const float lse = p.lse[r];
    float dl = pe * (g - acc);
    dl += p.aux_coef * (float)E / (float)p.T * pe * (frac - expected);
    dl += p.z_coef * 2.0f / (float)p.T * lse * pe;
    if (ev) p.dlogits[(int64_t)r * E + e] = dl;
}

// dWr = dlogits^T X is a GEMM with a long reduction (T rows) and a thin
// output (E x d), so it is split over row chunks.
// Pass 1: block (chunk, 256-column block, 16-expert block); lane l of every
// wave owns columns 4l..4l+3 of the block, wave w the rows w, w+4, ... of
// the chunk. Each wave accumulates 16 experts x 4 columns per lane over its
// rows in ascending order, with the X loads of the next 8 rows in flight;
// the four wave partials are then added in wave order through LDS.
constexpr int kDwExperts = 16;
constexpr int kDwCols = 256;
constexpr int kDwUnroll = 8;
constexpr int kDwRows = 256;  // most rows of one chunk (router_dw_chunks); 512 workgroups at c3
__global__ __launch_bounds__(kThreads) void router_dw_partial_kernel(RouterDwParams p) {
    __shared__ f32x4 s_part[3][kDwExperts][64];
    __shared__ f32x4 s_dl[kDwRows][kDwExperts / 4];  // the chunk's dlogits, experts e0 .. e0+15
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int chunk = blockIdx.x;
    const int col = blockIdx.y * kDwCols + lane * 4;
    const int e0 = blockIdx.z * kDwExperts;
    const int E = p.E, d = p.d;
    const int ne = min(kDwExperts, E - e0);
    const int rows_per = (p.T + p.nchunks - 1) / p.nchunks;  // <= kDwRows
    const int r0 = chunk * rows_per, r1 = min(p.T, r0 + rows_per);
    const int nr = max(0, r1 - r0);
    {
        // stage dlogits[r0 .. r1)[e0 .. e0+16) (zero past ne); loads issued first
        float* dst = reinterpret_cast<float*>(s_dl);
        constexpr int kPer = kDwRows * kDwExperts / kThreads;
        float v[kPer];
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int i = tid + u * kThreads, rr = i / kDwExperts, q = i % kDwExperts;
            const int r = r0 + min(rr, max(nr - 1, 0));
            v[u] = (rr < nr && q < ne) ? p.dlogits[(int64_t)r * E + e0 + min(q, ne - 1)] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kPer; ++u) dst[tid + u * kThreads] = v[u];
    }
    __syncthreads();
    const bool cok = col < d;
    const int ccol = cok ? col : 0;
    f32x4 acc[kDwExperts];
#pragma unroll
    for (int q = 0; q < kDwExperts; ++q) acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Two alternating 8-row register sets: the next batch's X loads are in
    // flight while the current batch is multiplied (addresses clamped to the
    // chunk's last row; rows past the chunk are skipped).
    auto xload = [&](int rb, uint2 (&xv)[kDwUnroll]) {
#pragma unroll
        for (int u = 0; u < kDwUnroll; ++u) {
            const int rr = min(rb + 4 * u, nr - 1);
            xv[u] = *reinterpret_cast<const uint2*>(p.X + (int64_t)(r0 + rr) * d + ccol);
        }
    };
    auto xmul = [&](int rb, const uint2 (&xv)[kDwUnroll]) {
#pragma unroll
        for (int u = 0; u < kDwUnroll; ++u) {
            const int rr = rb + 4 * u;
            if (rr >= nr) break;  // wave-uniform
            const float x0 = bf_lo(xv[u].x), x1 = bf_hi(xv[u].x), x2 = bf_lo(xv[u].y), x3 = bf_hi(xv[u].y);
#pragma unroll
            for (int q4 = 0; q4 < kDwExperts / 4; ++q4) {
                const f32x4 g4 = s_dl[rr][q4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const float g = g4[t];
                    acc[4 * q4 + t][0] += g * x0;
                    acc[4 * q4 + t][1] += g * x1;
                    acc[4 * q4 + t][2] += g * x2;
                    acc[4 * q4 + t][3] += g * x3;
                }
            }
        }
    };
    constexpr int kStep = 4 * kDwUnroll;  // rows of one batch over the four waves
    if (wave < nr) {  // uniform; an empty chunk (T == 0) loads nothing
        uint2 xa[kDwUnroll], xb[kDwUnroll];
        xload(wave, xa);
        for (int rb = wave; rb < nr; rb += 2 * kStep) {
            xload(rb + kStep, xb);
            xmul(rb, xa);
            if (rb + kStep >= nr) break;
            xload(rb + 2 * kStep, xa);
            xmul(rb + kStep, xb);
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int q = 0; q < kDwExperts; ++q) s_part[wave - 1][q][lane] = acc[q];
    }
    __syncthreads();
    if (wave == 0 && cok) {
#pragma unroll
        for (int q = 0; q < kDwExperts; ++q) {  // fixed trip count: acc stays in registers
            if (q < ne) {
                f32x4 v = acc[q];
                v += s_part[0][q][lane];
                v += s_part[1][q][lane];
                v += s_part[2][q][lane];
                *reinterpret_cast<f32x4*>(p.partial + ((int64_t)chunk * E + e0 + q) * d + col) = v;
            }
        }
    }
}

// Pass 1 on the matrix cores (d a multiple of 256, E a multiple of 4): the
// same (chunk, 256-column block) grid with experts in blocks of 32, the
// chunk's partial dWr[e][k] = sum_t dl[t][e] X[t][k] by
// v_mfma_f32_32x32x16_bf16 with the dlogits as src0 (expert rows) and X^T as
// src1 (column rows). The fp32 dlogits enter as two bf16 terms, hi =
// bf16(dl) and lo = bf16(dl - hi): both products with the bf16 X are exact
// in fp32, and hi + lo is within 2^-18 |dl| of dl, so the partial sums keep
// fp32 accuracy. Rows arrive in groups of 32 by DMA into three LDS buffers
// (X as [32][256] bf16 with the 16-byte chunks of odd rows at position
// XOR 4, the dlogits as [32][32] fp32); k step s of a group pairs lane half
// h with rows 16s + 2j + h (j = 0..7), so the two half-waves read rows of
// opposite parity and different banks. Wave w computes columns 64w .. 64w+63
// of the block (two 32-column tiles). Rows past the chunk enter as zeros.
constexpr int kDwmExperts = 32, kDwmGroup = 32, kDwmBufs = 3;
constexpr int kDwmXBytes = kDwmGroup * kDwCols * 2;         // 16 KiB
constexpr int kDwmBuf = kDwmXBytes + kDwmGroup * kDwmExperts * 4;  // + 4 KiB of dlogits
constexpr int kDwmLoads = 5;  // DMA loads per wave and group: 4 of X, 1 of dlogits
typedef float dwm_f32x16 __attribute__((ext_vector_type(16)));
template <int N>
__device__ __forceinline__ void dwm_wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__global__ __launch_bounds__(kThreads, 2) void router_dw_mfma_kernel(RouterDwParams p) {
    __shared__ uint4 s_buf[kDwmBufs * kDwmBuf / 16];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int chunk = blockIdx.x, c0 = blockIdx.y * kDwCols, e0 = blockIdx.z * kDwmExperts;
    const int E = p.E, d = p.d;
    const int rows_per = (p.T + p.nchunks - 1) / p.nchunks;  // <= kDwRows
    const int r0 = chunk * rows_per, r1 = min(p.T, r0 + rows_per);
    const int nr = max(0, r1 - r0);
    const int ng = (nr + kDwmGroup - 1) / kDwmGroup;
    const uint32_t sb = lds_u32(s_buf);
    const int h = lane >> 5, li = lane & 31;
    // Group g into buffer b: wave w loads X rows 8w .. 8w + 7 (two 512-byte
    // rows per load) and the dlogits rows 8w .. 8w + 7 (experts e0 .. e0+31,
    // 128 bytes per row). Rows past the chunk reload its last row, experts
    // past E the last four (both masked when read).
    auto dma_group = [&](int g, int b) {
        const uint32_t base = sb + (uint32_t)(b * kDwmBuf);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = wave * 4 + i, row = 2 * q + (lane >> 5), pos = lane & 31;
            const int rr = min(g * kDwmGroup + row, nr - 1);
            dma16_lds(p.X + (int64_t)(r0 + rr) * d + c0 + 8 * (pos ^ ((row & 1) * 4)), base + (uint32_t)q * 1024u);
        }
        const int row = 8 * wave + (lane >> 3), e = min(e0 + 4 * (lane & 7), E - 4);
        const int rr = min(g * kDwmGroup + row, nr - 1);
        dma16_lds(p.dlogits + (int64_t)(r0 + rr) * E + e, base + (uint32_t)(kDwmXBytes + wave * 1024));
    };
    dwm_f32x16 acc[2];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[c][r] = 0.0f;
#pragma unroll
    for (int g = 0; g < kDwmBufs - 1; ++g)
        if (g < ng) dma_group(g, g);
    for (int g = 0; g < ng; ++g) {
        // this wave's loads of group g are in once at most group g + 1's remain
        if (g + 1 < ng) dwm_wait_vm<kDwmLoads>();
        else dwm_wait_vm<0>();
        __syncthreads();  // every wave's loads of group g are in, and group g - 1's buffer is free
        if (g + kDwmBufs - 1 < ng) dma_group(g + kDwmBufs - 1, (g + kDwmBufs - 1) % kDwmBufs);
        const uint8_t* xb = reinterpret_cast<const uint8_t*>(s_buf) + (g % kDwmBufs) * kDwmBuf;
        const float* db = reinterpret_cast<const float*>(xb + kDwmXBytes);
        const int gr = g * kDwmGroup;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            float dv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int row = 16 * st + 2 * j + h;
                const float v = db[row * kDwmExperts + li];
                dv[j] = (gr + row < nr && e0 + li < E) ? v : 0.0f;
            }
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                hw[q] = pack_bf2(dv[2 * q], dv[2 * q + 1]);
                lw[q] = pack_bf2(dv[2 * q] - bf_lo(hw[q]), dv[2 * q + 1] - bf_hi(hw[q]));
            }
            const bf16x8 dh = __builtin_bit_cast(bf16x8, make_uint4(hw[0], hw[1], hw[2], hw[3]));
            const bf16x8 dlo = __builtin_bit_cast(bf16x8, make_uint4(lw[0], lw[1], lw[2], lw[3]));
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const int col = 64 * wave + 32 * ct + li;
                uint32_t xv[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int row = 16 * st + 2 * j + h;
                    const int pos = (col >> 3) ^ ((row & 1) * 4);
                    const uint32_t v = *reinterpret_cast<const uint16_t*>(xb + row * (kDwCols * 2) + pos * 16 + (col & 7) * 2);
                    xv[j] = gr + row < nr ? v : 0u;
                }
                const bf16x8 xf = __builtin_bit_cast(
                    bf16x8, make_uint4(xv[0] | (xv[1] << 16), xv[2] | (xv[3] << 16), xv[4] | (xv[5] << 16),
                                       xv[6] | (xv[7] << 16)));
                acc[ct] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(dh, xf, acc[ct], 0, 0, 0);
                acc[ct] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(dlo, xf, acc[ct], 0, 0, 0);
            }
        }
    }
    // acc[ct][r]: expert e0 + 8 (r / 4) + 4 h + r % 4, column c0 + 64 w + 32 ct + li
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int e = e0 + 8 * (r >> 2) + 4 * h + (r & 3);
            const int col = c0 + 64 * wave + 32 * ct + li;
            if (e < E && col < d) p.partial[((int64_t)chunk * E + e) * d + col] = acc[ct][r];
        }
}
static bool router_dw_mfma_fits(const RouterDwParams& p) {
    return p.d % kDwCols == 0 && p.E % 4 == 0 && p.E >= 4 && p.E <= kMaxExperts;
}

// Pass 2: dWr[e][k] = sum over chunks in ascending order; each thread owns
// one output and keeps 16 chunk loads in flight. Block b of the pass covers
// outputs [b * kThreads, (b + 1) * kThreads).
__device__ __forceinline__ void router_dw_reduce_block(const RouterDwParams& p, int b) {
    const int64_t n = (int64_t)p.E * p.d;
    const int64_t i = (int64_t)b * kThreads + threadIdx.x;
    if (i >= n) return;
    float s = 0.0f;
    int c = 0;
    for (; c + 16 <= p.nchunks; c += 16) {
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = p.partial[(int64_t)(c + u) * n + i];
#pragma unroll
        for (int u = 0; u < 16; ++u) s += v[u];
    }
    for (; c < p.nchunks; ++c) s += p.partial[(int64_t)c * n + i];
    p.dWr[i] = s;
}
__global__ __launch_bounds__(kThreads) void router_dw_reduce_kernel(RouterDwParams p) {
    router_dw_reduce_block(p, blockIdx.x);
}
int router_dw_reduce_blocks(const RouterDwParams& p) {
    return (int)(((int64_t)p.E * p.d + kThreads - 1) / kThreads);
}

// Gradient of one token row over the lane's 8 columns at c0: the K expert
// rows of dXg added in slot order, plus the router term sum_e dlogits_e Wr_e.
template <bool ROUTER>
__device__ __forceinline__ void scatter_chunk(const ScatterParams& p, const int* pos, const float* dl,
                                              const uint16_t* wl, int c0, float* acc) {
    const int d = p.d, K = p.K;
    uint4 xv[kMaxTopK];
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j)
        if (j < K) xv[j] = *reinterpret_cast<const uint4*>(p.dXg + (int64_t)pos[j] * d + c0);
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) {
        if (j < K) {
            float v[8];
            unpack8(xv[j], v);
#pragma unroll
            for (int t = 0; t < 8; ++t) acc[t] += v[t];
        }
    }
    if (ROUTER) {
        for (int e = 0; e < p.E; ++e) {
            const float g = dl[e];
            float w[8];
            unpack8(*reinterpret_cast<const uint4*>(wl + e * d + c0), w);
#pragma unroll
            for (int t = 0; t < 8; ++t) acc[t] += g * w[t];
        }
    }
}

// One wave per row. For the router input gradient, Wr and the block's rows
// of dlogits are staged in LDS (all loads of a thread issued before its LDS
// stores), so the per-expert loop reads only LDS.
//
// NI > 0 fuses the backward of the LayerNorm in front of the block
// (d <= 512*NI): the row's gradient dH = bf16(sum) stays in registers
// (rounded like the reference's bf16 dH), then
//   dS = rstd * ((g - mean(g)) - xh * mean(g * xh)),  g = dH * gamma,
//   xh = (S - mean) * rstd,
// and every lane keeps dgamma (dH * xh) and dbeta (dH) partials of its
// columns over the wave's rows (ascending); the four waves are added in
// order into one [2][d] partial per workgroup.
constexpr int kRedOnWrExperts = 12;  // E*d*2 bytes of Wr hold the 3*2*d floats
// WLDS: Wr is staged in LDS (router_wr_in_lds); otherwise it is read from
// global memory, with the same arithmetic.
template <bool ROUTER, int NI, bool WLDS>
__global__ __launch_bounds__(kThreads) void scatter_kernel(ScatterParams p, int rows_per_block) {
    extern __shared__ uint4 smem_w[];
    constexpr int NR = NI > 0 ? NI : 1;
    constexpr bool STAGE = ROUTER && WLDS;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int d = p.d, K = p.K, E = p.E;
    const int rbeg = blockIdx.x * rows_per_block;
    const int rend = min(p.T, rbeg + rows_per_block);
    float* s_dl = reinterpret_cast<float*>(smem_w + (STAGE ? E * d / 8 : 0));  // [rows_per_block][E]
    // [3][2][d] wave partials of the LayerNorm variant: over the staged Wr
    // once every wave is done with it (E >= 12), else after the dlogits.
    const bool red_on_wr = STAGE && E >= kRedOnWrExperts;
    float* s_red = red_on_wr ? reinterpret_cast<float*>(smem_w) : s_dl + (ROUTER ? rows_per_block * E : 0);
    if (ROUTER) {
        if (STAGE) {
            const uint4* src = reinterpret_cast<const uint4*>(p.Wr);
            const int nvec = E * d / 8;
            for (int i0 = threadIdx.x; i0 < nvec; i0 += 8 * kThreads) {
                uint4 v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = src[min(i0 + u * kThreads, nvec - 1)];
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (i0 + u * kThreads < nvec) smem_w[i0 + u * kThreads] = v[u];
            }
        }
        const int ndl = (rend - rbeg) * E;
        for (int i = threadIdx.x; i < ndl; i += kThreads) s_dl[i] = p.dlogits[(int64_t)rbeg * E + i];
        __syncthreads();
    }
    const uint16_t* wl = STAGE ? reinterpret_cast<const uint16_t*>(smem_w) : p.Wr;

    float gam[NR][8], pg[NR][8], pb[NR][8];
    if constexpr (NI > 0) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int c0 = i * 512 + lane * 8;
            f32x4 g0 = f32x4{0.f, 0.f, 0.f, 0.f}, g1 = g0;
            if (c0 < d) {
                g0 = *reinterpret_cast<const f32x4*>(p.ln_gamma + c0);
                g1 = *reinterpret_cast<const f32x4*>(p.ln_gamma + c0 + 4);
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                gam[i][t] = g0[t];
                gam[i][t + 4] = g1[t];
            }
#pragma unroll
            for (int t = 0; t < 8; ++t) pg[i][t] = pb[i][t] = 0.0f;
        }
    }

    for (int r = rbeg + wave; r < rend; r += 4) {
        int pos[kMaxTopK];
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j)
            if (j < K) pos[j] = p.slot_of[(int64_t)r * K + j];
        const float* dl = s_dl + (r - rbeg) * E;
        if constexpr (NI == 0) {
            for (int c0 = lane * 8; c0 < d; c0 += 512) {
                float acc[8];
                scatter_chunk<ROUTER>(p, pos, dl, wl, c0, acc);
                *reinterpret_cast<uint4*>(p.dX + (int64_t)r * d + c0) = pack8(acc);
            }
        } else {
            const float mean = p.ln_mean[r], rstd = p.ln_rstd[r];
            float hv[NI][8], xs[NI][8];
            float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int c0 = i * 512 + lane * 8;
                if (c0 < d) {
                    const uint4 sv = *reinterpret_cast<const uint4*>(p.ln_S + (int64_t)r * d + c0);
                    float acc[8];
                    scatter_chunk<ROUTER>(p, pos, dl, wl, c0, acc);
                    unpack8(pack8(acc), hv[i]);
                    unpack8(sv, xs[i]);
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        const float g = hv[i][t] * gam[i][t];
                        const float xh = (xs[i][t] - mean) * rstd;
                        s1 += g;
                        s2 += g * xh;
                        pg[i][t] += hv[i][t] * xh;
                        pb[i][t] += hv[i][t];
                    }
                }
            }
            s1 = wave_sum(s1);
            s2 = wave_sum(s2);
            const float a = s1 / (float)d, b = s2 / (float)d;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int c0 = i * 512 + lane * 8;
                if (c0 < d) {
                    float out[8];
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        const float g = hv[i][t] * gam[i][t];
                        const float xh = (xs[i][t] - mean) * rstd;
                        out[t] = rstd * ((g - a) - xh * b);
                    }
                    *reinterpret_cast<uint4*>(p.ln_dS + (int64_t)r * d + c0) = pack8(out);
                }
            }
        }
    }

    if constexpr (NI > 0) {
        if (red_on_wr) __syncthreads();  // Wr reads done before it is overwritten
        if (wave > 0) {
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int c0 = i * 512 + lane * 8;
                if (c0 < d) {
                    float* dg = s_red + (int64_t)((wave - 1) * 2) * d + c0;
                    float* db = dg + d;
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        dg[t] = pg[i][t];
                        db[t] = pb[i][t];
                    }
                }
            }
        }
        __syncthreads();
        if (wave == 0) {
            float* outg = p.ln_partial + (int64_t)blockIdx.x * 2 * d;
            float* outb = outg + d;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int c0 = i * 512 + lane * 8;
                if (c0 < d) {
                    float g[8], b[8];
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        g[t] = ((pg[i][t] + s_red[c0 + t]) + s_red[2 * d + c0 + t]) + s_red[4 * d + c0 + t];
                        b[t] = ((pb[i][t] + s_red[d + c0 + t]) + s_red[3 * d + c0 + t]) + s_red[5 * d + c0 + t];
                    }
                    *reinterpret_cast<f32x4*>(outg + c0) = f32x4{g[0], g[1], g[2], g[3]};
                    *reinterpret_cast<f32x4*>(outg + c0 + 4) = f32x4{g[4], g[5], g[6], g[7]};
                    *reinterpret_cast<f32x4*>(outb + c0) = f32x4{b[0], b[1], b[2], b[3]};
                    *reinterpret_cast<f32x4*>(outb + c0 + 4) = f32x4{b[4], b[5], b[6], b[7]};
                }
            }
        }
    }
}

}  // namespace

hipError_t launch_combine(const CombineParams& p, hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    if (p.self_dispatch && (p.T > kSkinnyMaxTokens || p.idx == nullptr)) return hipErrorInvalidValue;
    const int grid = (p.T + 3) / 4 + (p.self_dispatch ? 1 : 0);
    if (p.part != nullptr) {
        if (p.silu || p.O_out == nullptr || p.slots != p.T * p.K) return hipErrorInvalidValue;
        switch (p.K) {
            case 1: combine_part_kernel<1><<<grid, kThreads, 0, s>>>(p); break;
            case 2: combine_part_kernel<2><<<grid, kThreads, 0, s>>>(p); break;
            case 3: combine_part_kernel<3><<<grid, kThreads, 0, s>>>(p); break;
            case 4: combine_part_kernel<4><<<grid, kThreads, 0, s>>>(p); break;
            case 5: combine_part_kernel<5><<<grid, kThreads, 0, s>>>(p); break;
            case 6: combine_part_kernel<6><<<grid, kThreads, 0, s>>>(p); break;
            case 7: combine_part_kernel<7><<<grid, kThreads, 0, s>>>(p); break;
            case 8: combine_part_kernel<8><<<grid, kThreads, 0, s>>>(p); break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    switch (p.K * 2 + (p.silu ? 1 : 0)) {
#define TMT_COMBINE(KK)                                                       \
    case 2 * KK: combine_kernel<false, KK><<<grid, kThreads, 0, s>>>(p); break; \
    case 2 * KK + 1: combine_kernel<true, KK><<<grid, kThreads, 0, s>>>(p); break;
        TMT_COMBINE(1)
        TMT_COMBINE(2)
        TMT_COMBINE(3)
        TMT_COMBINE(4)
        TMT_COMBINE(5)
        TMT_COMBINE(6)
        TMT_COMBINE(7)
        TMT_COMBINE(8)
#undef TMT_COMBINE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_combine_bwd(const CombineBwdParams& p, hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    const int grid = (p.T + 3) / 4;
    switch (p.K * 2 + (p.silu ? 1 : 0)) {
#define TMT_COMBINE_BWD(KK)                                                       \
    case 2 * KK: combine_bwd_kernel<false, KK><<<grid, kThreads, 0, s>>>(p); break; \
    case 2 * KK + 1: combine_bwd_kernel<true, KK><<<grid, kThreads, 0, s>>>(p); break;
        TMT_COMBINE_BWD(1)
        TMT_COMBINE_BWD(2)
        TMT_COMBINE_BWD(3)
        TMT_COMBINE_BWD(4)
        TMT_COMBINE_BWD(5)
        TMT_COMBINE_BWD(6)
        TMT_COMBINE_BWD(7)
        TMT_COMBINE_BWD(8)
#undef TMT_COMBINE_BWD
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Row chunks of pass 1: at most kDwRows rows each (the LDS-staged dlogits
// block), and, where T is small, enough chunks that the pass has about
// kDwMinBlocks workgroups (chunks of at least kDwMinRows rows). More chunks
// shorten pass 1 and lengthen pass 2's per-output sums: at the reference's
// profile shape (T = 2048, d = 1280, E = 8) 256 workgroups took 12.8 us for
// both passes against 14.2 us with 128 and 16.9 us with 512.
constexpr int kDwMinBlocks = 256, kDwMinRows = 16;
static int router_dw_blocks_per_chunk(int E, int d) {
    return ((d + kDwCols - 1) / kDwCols) * ((E + kDwExperts - 1) / kDwExperts);
}
int router_dw_chunks(int T, int E, int d) {
    if (T <= 0) return 1;
    const int want = (kDwMinBlocks + router_dw_blocks_per_chunk(E, d) - 1) / router_dw_blocks_per_chunk(E, d);
    int rows = (T + want - 1) / want;
    rows = rows < kDwMinRows ? kDwMinRows : rows > kDwRows ? kDwRows : rows;
    return (T + rows - 1) / rows;
}
// router_dw_chunks(T, E, d) <= this for every T <= max_tokens: chunks of
// fewer than kDwRows rows number at most `want`, full-size chunks at most
// ceil(max_tokens / kDwRows).
int router_dw_chunks_max(int max_tokens, int E, int d) {
    const int want = (kDwMinBlocks + router_dw_blocks_per_chunk(E, d) - 1) / router_dw_blocks_per_chunk(E, d);
    const int c = (max_tokens + kDwRows - 1) / kDwRows;
    return std::max(1, std::max(c, want));
}

hipError_t launch_router_dw(const RouterDwParams& p, hipStream_t s, bool reduce) {
    if (p.nchunks < 1 || (int64_t)p.nchunks * kDwRows < p.T) return hipErrorInvalidValue;
    if (router_dw_mfma_fits(p)) {
        dim3 grid1(p.nchunks, p.d / kDwCols, (p.E + kDwmExperts - 1) / kDwmExperts);
        router_dw_mfma_kernel<<<grid1, kThreads, 0, s>>>(p);
    } else {
        dim3 grid1(p.nchunks, (p.d + kDwCols - 1) / kDwCols, (p.E + kDwExperts - 1) / kDwExperts);
        router_dw_partial_kernel<<<grid1, kThreads, 0, s>>>(p);
    }
    if (reduce) router_dw_reduce_kernel<<<(unsigned)router_dw_reduce_blocks(p), kThreads, 0, s>>>(p);
    return hipGetLastError();
}

// Variant without the LayerNorm: each wave keeps RPW rows in flight (rows
// w, w + 4, ..., of the workgroup's slice in groups of RPW): the K gathered
// dXg chunks of all RPW rows are loaded together, and each staged Wr chunk is
// unpacked once for the RPW rows. K is a template argument so that every
// load is issued unconditionally. Per row the sum runs in the same order as
// scatter_chunk (picks j ascending, then experts e ascending).
namespace {
constexpr int kScatterRowsPerWave = 4;
// Rows per workgroup of the router variant: 32 gives 1024 workgroups at
// T = 32768, four per CU (LDS: E*d*2 bytes of Wr + 32*E*4 of dlogits).
constexpr int kScatterRowsRouter = 32;
constexpr int kScatterRowsRouterMin = 8;
template <bool ROUTER, int K, bool WLDS>
__global__ __launch_bounds__(kThreads) void scatter_rows_kernel(ScatterParams p, int rows_per_block) {
    extern __shared__ uint4 smem_w[];
    constexpr int RPW = kScatterRowsPerWave;
    constexpr bool STAGE = ROUTER && WLDS;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int d = p.d, E = p.E;
    const int nrow_blocks = (p.T + rows_per_block - 1) / rows_per_block;
    if ((int)blockIdx.x >= nrow_blocks) {  // the router weight gradient's pass 2
        router_dw_reduce_block(p.dw, blockIdx.x - nrow_blocks);
        return;
    }
    const int rbeg = blockIdx.x * rows_per_block;
    const int rend = min(p.T, rbeg + rows_per_block);
    float* s_dl = reinterpret_cast<float*>(smem_w + (STAGE ? E * d / 8 : 0));  // [rows_per_block][E]
    if (ROUTER) {
        if (STAGE) {
            const uint4* src = reinterpret_cast<const uint4*>(p.Wr);
            const int nvec = E * d / 8;
            for (int i0 = threadIdx.x; i0 < nvec; i0 += 8 * kThreads) {
                uint4 v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = src[min(i0 + u * kThreads, nvec - 1)];
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (i0 + u * kThreads < nvec) smem_w[i0 + u * kThreads] = v[u];
            }
        }
        const int ndl = (rend - rbeg) * E;
        for (int i = threadIdx.x; i < ndl; i += kThreads) s_dl[i] = p.dlogits[(int64_t)rbeg * E + i];
        __syncthreads();
    }
    const uint16_t* wl = STAGE ? reinterpret_cast<const uint16_t*>(smem_w) : p.Wr;
    for (int r = rbeg + wave; r < rend; r += 4 * RPW) {
        int row[RPW], pos[RPW][K];
        bool ok[RPW];
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            ok[i] = r + 4 * i < rend;
            row[i] = ok[i] ? r + 4 * i : r;  // clamped: a row past the slice is loaded, not stored
#pragma unroll
            for (int j = 0; j < K; ++j) pos[i][j] = p.slot_of[(int64_t)row[i] * K + j];
        }
        for (int c0 = lane * 8; c0 < d; c0 += 512) {
            uint4 xv[RPW][K];
#pragma unroll
            for (int i = 0; i < RPW; ++i)
#pragma unroll
                for (int j = 0; j < K; ++j) xv[i][j] = *reinterpret_cast<const uint4*>(p.dXg + (int64_t)pos[i][j] * d + c0);
            float acc[RPW][8];
#pragma unroll
            for (int i = 0; i < RPW; ++i) {
#pragma unroll
                for (int t = 0; t < 8; ++t) acc[i][t] = 0.0f;
#pragma unroll
                for (int j = 0; j < K; ++j) {
                    float v[8];
                    unpack8(xv[i][j], v);
#pragma unroll
                    for (int t = 0; t < 8; ++t) acc[i][t] += v[t];
                }
            }
            if (ROUTER) {
                for (int e = 0; e < E; ++e) {
                    float w[8];
                    unpack8(*reinterpret_cast<const uint4*>(wl + e * d + c0), w);
#pragma unroll
                    for (int i = 0; i < RPW; ++i) {
                        const float g = s_dl[(row[i] - rbeg) * E + e];
#pragma unroll
                        for (int t = 0; t < 8; ++t) acc[i][t] += g * w[t];
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < RPW; ++i)
                if (ok[i]) *reinterpret_cast<uint4*>(p.dX + (int64_t)row[i] * d + c0) = pack8(acc[i]);
        }
    }
}
// LayerNorm variant with two rows per wave in flight (rows r and r + 4 of
// the wave's stride; K and the chunk count are template arguments so that
// both rows' loads are issued unconditionally): each staged Wr chunk is
// unpacked once for the two rows. Per row the arithmetic is scatter_kernel's
// (picks j ascending, then experts e ascending; dgamma / dbeta partials over
// the wave's rows in ascending order), so the results are bit-identical.
template <int K, int NI, bool WLDS>
__global__ __launch_bounds__(kThreads) void scatter_ln2_kernel(ScatterParams p, int rows_per_block) {
    extern __shared__ uint4 smem_w[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int d = p.d, E = p.E;
    const int rbeg = blockIdx.x * rows_per_block;
    const int rend = min(p.T, rbeg + rows_per_block);
    float* s_dl = reinterpret_cast<float*>(smem_w + (WLDS ? E * d / 8 : 0));  // [rows_per_block][E]
    const bool red_on_wr = WLDS && E >= kRedOnWrExperts;
    float* s_red = red_on_wr ? reinterpret_cast<float*>(smem_w) : s_dl + rows_per_block * E;
    if (WLDS) {
        const uint4* src = reinterpret_cast<const uint4*>(p.Wr);
        const int nvec = E * d / 8;
        for (int i0 = threadIdx.x; i0 < nvec; i0 += 8 * kThreads) {
            uint4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = src[min(i0 + u * kThreads, nvec - 1)];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (i0 + u * kThreads < nvec) smem_w[i0 + u * kThreads] = v[u];
        }
    }
    {
        const int ndl = (rend - rbeg) * E;
        for (int i = threadIdx.x; i < ndl; i += kThreads) s_dl[i] = p.dlogits[(int64_t)rbeg * E + i];
    }
    __syncthreads();
    const uint16_t* wl = WLDS ? reinterpret_cast<const uint16_t*>(smem_w) : p.Wr;

    float gam[NI][8], pg[NI][8], pb[NI][8];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int c0 = i * 512 + lane * 8;
        f32x4 g0 = f32x4{0.f, 0.f, 0.f, 0.f}, g1 = g0;
        if (c0 < d) {
            g0 = *reinterpret_cast<const f32x4*>(p.ln_gamma + c0);
            g1 = *reinterpret_cast<const f32x4*>(p.ln_gamma + c0 + 4);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            gam[i][t] = g0[t];
            gam[i][t + 4] = g1[t];
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) pg[i][t] = pb[i][t] = 0.0f;
    }

    for (int r = rbeg + wave; r < rend; r += 8) {
        const bool two = r + 4 < rend;  // wave-uniform
        int row[2], pos[2][K];
        row[0] = r;
        row[1] = two ? r + 4 : r;  // clamped: the second row is loaded but not used
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int j = 0; j < K; ++j) pos[q][j] = p.slot_of[(int64_t)row[q] * K + j];
        float mean[2], rstd[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            mean[q] = p.ln_mean[row[q]];
            rstd[q] = p.ln_rstd[row[q]];
        }
        float hv[2][NI][8], xs[2][NI][8];
        float s1[2] = {0.0f, 0.0f}, s2[2] = {0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int c0 = i * 512 + lane * 8;
            if (c0 < d) {
                uint4 xv[2][K], sv[2];
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    sv[q] = *reinterpret_cast<const uint4*>(p.ln_S + (int64_t)row[q] * d + c0);
#pragma unroll
                    for (int j = 0; j < K; ++j) xv[q][j] = *reinterpret_cast<const uint4*>(p.dXg + (int64_t)pos[q][j] * d + c0);
                }
                float acc[2][8];
#pragma unroll
                for (int q = 0; q < 2; ++q) {
#pragma unroll
                    for (int t = 0; t < 8; ++t) acc[q][t] = 0.0f;
#pragma unroll
                    for (int j = 0; j < K; ++j) {
                        float v[8];
                        unpack8(xv[q][j], v);
#pragma unroll
                        for (int t = 0; t < 8; ++t) acc[q][t] += v[t];
                    }
                }
                const float* dl0 = s_dl + (row[0] - rbeg) * E;
                const float* dl1 = s_dl + (row[1] - rbeg) * E;
                for (int e = 0; e < E; ++e) {
                    const float g0 = dl0[e], g1 = dl1[e];
                    float w[8];
                    unpack8(*reinterpret_cast<const uint4*>(wl + e * d + c0), w);
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        acc[0][t] += g0 * w[t];
                        acc[1][t] += g1 * w[t];
                    }
                }
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    unpack8(pack8(acc[q]), hv[q][i]);
                    unpack8(sv[q], xs[q][i]);
                    if (q == 0 || two) {
#pragma unroll
                        for (int t = 0; t < 8; ++t) {
                            const float g = hv[q][i][t] * gam[i][t];
                            const float xh = (xs[q][i][t] - mean[q]) * rstd[q];
                            s1[q] += g;
                            s2[q] += g * xh;
                            pg[i][t] += hv[q][i][t] * xh;
                            pb[i][t] += hv[q][i][t];
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            if (q == 1 && !two) break;  // wave-uniform
            const float a = wave_sum(s1[q]) / (float)d, b = wave_sum(s2[q]) / (float)d;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int c0 = i * 512 + lane * 8;
                if (c0 < d) {
                    float out[8];
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        const float g = hv[q][i][t] * gam[i][t];
                        const float xh = (xs[q][i][t] - mean[q]) * rstd[q];
                        out[t] = rstd[q] * ((g - a) - xh * b);
                    }
                    *reinterpret_cast<uint4*>(p.ln_dS + (int64_t)row[q] * d + c0) = pack8(out);
                }
            }
        }
    }

    if (red_on_wr) __syncthreads();  // Wr reads done before it is overwritten
    if (wave > 0) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int c0 = i * 512 + lane * 8;
            if (c0 < d) {
                float* dg = s_red + (int64_t)((wave - 1) * 2) * d + c0;
                float* db = dg + d;
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    dg[t] = pg[i][t];
                    db[t] = pb[i][t];
                }
            }
        }
    }
    __syncthreads();
    if (wave == 0) {
        float* outg = p.ln_partial + (int64_t)blockIdx.x * 2 * d;
        float* outb = outg + d;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int c0 = i * 512 + lane * 8;
            if (c0 < d) {
                float g[8], b[8];
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    g[t] = ((pg[i][t] + s_red[c0 + t]) + s_red[2 * d + c0 + t]) + s_red[4 * d + c0 + t];
                    b[t] = ((pb[i][t] + s_red[d + c0 + t]) + s_red[3 * d + c0 + t]) + s_red[5 * d + c0 + t];
                }
                *reinterpret_cast<f32x4*>(outg + c0) = f32x4{g[0], g[1], g[2], g[3]};
                *reinterpret_cast<f32x4*>(outg + c0 + 4) = f32x4{g[4], g[5], g[6], g[7]};
                *reinterpret_cast<f32x4*>(outb + c0) = f32x4{b[0], b[1], b[2], b[3]};
                *reinterpret_cast<f32x4*>(outb + c0 + 4) = f32x4{b[4], b[5], b[6], b[7]};
            }
        }
    }
}

}  // namespace

int scatter_blocks(int T) {
    const int b = (T + kScatterRows - 1) / kScatterRows;
    return b < 1 ? 1 : b;
}

template <bool ROUTER, bool WLDS>
hipError_t launch_scatter_ni(const ScatterParams& p, int ni, int rows, size_t lds, hipStream_t s) {
    const int grid = (p.T + rows - 1) / rows;
    switch (ni) {
        case 0: scatter_kernel<ROUTER, 0, WLDS><<<grid, kThreads, lds, s>>>(p, rows); break;
        case 1: scatter_kernel<ROUTER, 1, WLDS><<<grid, kThreads, lds, s>>>(p, rows); break;
        case 2: scatter_kernel<ROUTER, 2, WLDS><<<grid, kThreads, lds, s>>>(p, rows); break;
        case 3: scatter_kernel<ROUTER, 3, WLDS><<<grid, kThreads, lds, s>>>(p, rows); break;
        case 4: scatter_kernel<ROUTER, 4, WLDS><<<grid, kThreads, lds, s>>>(p, rows); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

namespace {
__global__ __launch_bounds__(kThreads) void zero_f32_kernel(float* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
        p[i] = 0.0f;
}
}  // namespace

namespace {
__global__ __launch_bounds__(kThreads) void f32_to_bf16_kernel(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
        out[i] = f2bf(in[i]);
}
}  // namespace

hipError_t launch_f32_to_bf16(const float* in, uint16_t* out, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((n + kThreads - 1) / kThreads, 4096);
    f32_to_bf16_kernel<<<(unsigned)blocks, kThreads, 0, s>>>(in, out, n);
    return hipGetLastError();
}

namespace {
// One thread per destination element (these copies serve widths that are not
// a multiple of 64, where speed is not the point).
template <typename V>
__global__ __launch_bounds__(kThreads) void pad_copy_kernel(PadParams p) {
    const V* src = static_cast<const V*>(p.src[blockIdx.y]);
    V* dst = static_cast<V*>(p.dst[blockIdx.y]);
    const int64_t n = p.rows_d * p.cols_d;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
        const int64_t r = i / p.cols_d, c = i - r * p.cols_d;
        V v = 0;
        if (r < p.rows_s && c < p.cols_s) v = src[r * p.ld_s + c];
        dst[r * p.ld_d + c] = v;
    }
}
}  // namespace

hipError_t launch_pad_copy(const PadParams& p, int nmat, int elem_bytes, hipStream_t s) {
    if (nmat < 0 || nmat > kMaxExperts || p.cols_s > p.ld_s || p.cols_d > p.ld_d) return hipErrorInvalidValue;
    const int64_t n = p.rows_d * p.cols_d;
    if (nmat == 0 || n <= 0) return hipSuccess;
    const unsigned blocks = (unsigned)std::min<int64_t>((n + kThreads - 1) / kThreads, 2048);
    if (elem_bytes == 2) pad_copy_kernel<uint16_t><<<dim3(blocks, nmat), kThreads, 0, s>>>(p);
    else if (elem_bytes == 4) pad_copy_kernel<float><<<dim3(blocks, nmat), kThreads, 0, s>>>(p);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

namespace {
// dst[e] = src[e]^T for bf16 matrices [rows][cols] -> [cols][rows], through
// 64 x 64 LDS tiles: 16-byte loads along the source rows, 16-byte stores
// along the destination rows (both coalesced), one tile per workgroup.
__global__ __launch_bounds__(kThreads) void transpose_bf16_kernel(TransposeParams p) {
    __shared__ uint16_t t[64][64 + 2];
    const int e = blockIdx.z;
    const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
    const uint16_t* src = p.src[e];
    uint16_t* dst = p.dst + (int64_t)e * p.rows * p.cols;
    const int tx = threadIdx.x & 7, ty = threadIdx.x >> 3;  // 8 lanes x 16 bytes per 64-element row
    uint4 v[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = r0 + ty + 32 * i;
        v[i] = r < p.rows ? *reinterpret_cast<const uint4*>(src + (int64_t)r * p.ld_src + c0 + tx * 8) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            t[ty + 32 * i][tx * 8 + 2 * q] = (uint16_t)(w[q] & 0xffff);
            t[ty + 32 * i][tx * 8 + 2 * q + 1] = (uint16_t)(w[q] >> 16);
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = ty + 32 * i;  // destination row (source column c0 + c)
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            w[q] = (uint32_t)t[tx * 8 + 2 * q][c] | ((uint32_t)t[tx * 8 + 2 * q + 1][c] << 16);
        const int rr = r0 + tx * 8;  // destination columns rr .. rr + 7
        if (c0 + c < p.cols && rr < p.rows)
            *reinterpret_cast<uint4*>(dst + (int64_t)(c0 + c) * p.rows + rr) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}
}  // namespace

hipError_t launch_transpose_bf16(const TransposeParams& p, int nmat, hipStream_t s) {
    if (nmat < 0 || nmat > kMaxExperts || p.rows % 64 != 0 || p.cols % 64 != 0 || p.ld_src < p.cols)
        return hipErrorInvalidValue;
    if (nmat == 0 || p.rows == 0 || p.cols == 0) return hipSuccess;
    transpose_bf16_kernel<<<dim3(p.cols / 64, p.rows / 64, nmat), kThreads, 0, s>>>(p);
    return hipGetLastError();
}

hipError_t launch_zero_f32(float* p, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((n + kThreads - 1) / kThreads, 1024);
    zero_f32_kernel<<<(unsigned)blocks, kThreads, 0, s>>>(p, n);
    return hipGetLastError();
}

hipError_t launch_scatter(const ScatterParams& p, hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    if (p.dw.partial != nullptr && (p.ln_S != nullptr || p.dw.nchunks < 1)) return hipErrorInvalidValue;
    const bool router = p.dlogits != nullptr && p.E > 1;
    const bool ln = p.ln_S != nullptr;
    if (ln && p.d > kLnFusedMaxD) return hipErrorInvalidValue;
    const int rows = (router || ln) ? kScatterRows : 4;
    const bool wlds = router && router_wr_in_lds(p.E, p.d);  // Wr staged in LDS
    const size_t wr_lds = wlds ? (size_t)p.E * p.d * 2 : 0;
    size_t lds = router ? wr_lds + (size_t)rows * p.E * 4 : 0;
    if (ln && !(wlds && p.E >= kRedOnWrExperts)) lds += (size_t)3 * 2 * p.d * 4;
    const int ni = ln ? (p.d + 511) / 512 : 0;
    if (ni == 0) {
        // router variant: fewer rows per workgroup while that keeps the grid
        // under 512 workgroups (small T: each wave's chain of chunk loads is
        // the time, so more, shorter workgroups finish sooner)
        int rrows = router ? kScatterRowsRouter : 4 * kScatterRowsPerWave;
        while (router && rrows > kScatterRowsRouterMin && (p.T + rrows - 1) / rrows < 512) rrows /= 2;
        // pass 2 of the router weight gradient rides along (extra workgroups)
        const int grid = (p.T + rrows - 1) / rrows + (p.dw.partial != nullptr ? router_dw_reduce_blocks(p.dw) : 0);
        const size_t rlds = router ? wr_lds + (size_t)rrows * p.E * 4 : 0;
        switch (p.K * 2 + (router ? 1 : 0)) {
#define TMT_SCATTER_ROWS(KK)                                                                   \
    case 2 * KK: scatter_rows_kernel<false, KK, false><<<grid, kThreads, 0, s>>>(p, rrows); break; \
    case 2 * KK + 1:                                                                           \
        if (wlds) scatter_rows_kernel<true, KK, true><<<grid, kThreads, rlds, s>>>(p, rrows);    \
        else scatter_rows_kernel<true, KK, false><<<grid, kThreads, rlds, s>>>(p, rrows);        \
        break;
            TMT_SCATTER_ROWS(1)
            TMT_SCATTER_ROWS(2)
            TMT_SCATTER_ROWS(3)
            TMT_SCATTER_ROWS(4)
            TMT_SCATTER_ROWS(5)
            TMT_SCATTER_ROWS(6)
            TMT_SCATTER_ROWS(7)
            TMT_SCATTER_ROWS(8)
#undef TMT_SCATTER_ROWS
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    if (!router) return launch_scatter_ni<false, false>(p, ni, rows, lds, s);
    if (p.K <= 4 && ni <= 2) {
        // two rows per wave in flight (scatter_ln2_kernel)
        const int grid = (p.T + rows - 1) / rows;
#define TMT_LN2(KK, NN)                                                                                    \
    if (p.K == KK && ni == NN) {                                                                          \
        if (wlds) scatter_ln2_kernel<KK, NN, true><<<grid, kThreads, lds, s>>>(p, rows);                   \
        else scatter_ln2_kernel<KK, NN, false><<<grid, kThreads, lds, s>>>(p, rows);                       \
        return hipGetLastError();                                                                         \
    }
        TMT_LN2(1, 1) TMT_LN2(2, 1) TMT_LN2(3, 1) TMT_LN2(4, 1)
        TMT_LN2(1, 2) TMT_LN2(2, 2) TMT_LN2(3, 2) TMT_LN2(4, 2)
#undef TMT_LN2
    }
    return wlds ? launch_scatter_ni<true, true>(p, ni, rows, lds, s)
                : launch_scatter_ni<true, false>(p, ni, rows, lds, s);
}

}  // namespace tmt
