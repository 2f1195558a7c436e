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
#include "device_util.hpp"
#include "moe_internal.hpp"

namespace tmt {
namespace {

template <bool SILU>
__global__ __launch_bounds__(kThreads) void combine_kernel(CombineParams p) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= p.T) return;
    const int d = p.d, K = p.K;
    int pos[kMaxTopK];
    float g[kMaxTopK];
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) {
        if (j < K) {
            pos[j] = p.slot_of[(int64_t)r * K + j];
            g[j] = p.gate[(int64_t)r * K + j];
        }
    }
    for (int c0 = lane * 8; c0 < d; c0 += 512) {
        float acc[8];
        uint4* yp = reinterpret_cast<uint4*>(p.Y + (int64_t)r * d + c0);
        if (p.beta != 0.0f) {
            unpack8(*yp, acc);
#pragma unroll
            for (int t = 0; t < 8; ++t) acc[t] *= p.beta;
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) acc[t] = 0.0f;
        }
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j) {
            if (j < K) {
                float o[8];
                unpack8(*reinterpret_cast<const uint4*>(p.O + (int64_t)pos[j] * d + c0), o);
#pragma unroll
                for (int t = 0; t < 8; ++t) acc[t] += g[j] * (SILU ? silu_fast(o[t]) : o[t]);
            }
        }
        *yp = pack8(acc);
    }
}

template <bool SILU>
__global__ __launch_bounds__(kThreads) void combine_bwd_kernel(CombineBwdParams p) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= p.T) return;
    const int d = p.d, K = p.K, E = p.E;
    float s[kMaxTopK];
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) {
        if (j < K) {
            const int64_t pos = p.slot_of[(int64_t)r * K + j];
            const float g = p.gate[(int64_t)r * K + j];
            float part = 0.0f;
            for (int c0 = lane * 8; c0 < d; c0 += 512) {
                float dy[8], o[8], out[8];
                unpack8(*reinterpret_cast<const uint4*>(p.dY + (int64_t)r * d + c0), dy);
                unpack8(*reinterpret_cast<const uint4*>(p.O + pos * d + c0), o);
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    if (SILU) {
                        // Reference experts: gradient through the SiLU applied in
                        // combine (combine_bwd_kernel, moe.cu:162-176).
                        part += dy[t] * silu_fast(o[t]);
                        out[t] = g * dy[t] * dsilu_fast(o[t]);
                    } else {
                        part += dy[t] * o[t];
                        out[t] = g * dy[t];
                    }
                }
                *reinterpret_cast<uint4*>(p.dO + pos * d + c0) = pack8(out);
                *reinterpret_cast<uint4*>(p.Xg + pos * d + c0) =
                    *reinterpret_cast<const uint4*>(p.X + (int64_t)r * d + c0);
            }
            s[j] = wave_sum(part);
        }
    }
    if (E <= 1) return;

    // Router backward for row r, lane e (router_bwd_kernel, moe.cu:199-234).
    const int e = lane;
    const bool ev = e < E;
    const float pe = ev ? p.probs[(int64_t)r * E + e] : 0.0f;
    float Z = 0.0f, sp = 0.0f, g = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) {
        if (j < K) {
            const int ej = p.idx[(int64_t)r * K + j];
            const float pj = p.probs[(int64_t)r * E + ej];
            Z += pj;
            sp += s[j] * pj;
        }
    }
    const float Z2 = Z * Z + 1e-12f;
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) {
        if (j < K && p.idx[(int64_t)r * K + j] == e) g = (s[j] * Z - sp) / Z2;
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

// Pass 1: block (chunk, column block, expert block) accumulates 16 experts x
// 4 columns per thread over its rows in ascending order.
constexpr int kDwExperts = 16;
__global__ __launch_bounds__(kThreads) void router_dw_partial_kernel(RouterDwParams p) {
    __shared__ float s_dl[64][kDwExperts];
    const int tid = threadIdx.x;
    const int chunk = blockIdx.x;
    const int col = blockIdx.y * 1024 + tid * 4;
    const int e0 = blockIdx.z * kDwExperts;
    const int E = p.E, d = p.d;
    const int ne = min(kDwExperts, E - e0);
    const int rows_per = (p.T + p.nchunks - 1) / p.nchunks;
    const int r0 = chunk * rows_per, r1 = min(p.T, r0 + rows_per);
    float acc[kDwExperts][4];
#pragma unroll
    for (int q = 0; q < kDwExperts; ++q)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[q][t] = 0.0f;
    for (int rb = r0; rb < r1; rb += 64) {
        const int nr = min(64, r1 - rb);
        __syncthreads();
        for (int i = tid; i < 64 * kDwExperts; i += kThreads) {
            const int rr = i / kDwExperts, q = i % kDwExperts;
            s_dl[rr][q] = (rr < nr && q < ne) ? p.dlogits[(int64_t)(rb + rr) * E + e0 + q] : 0.0f;
        }
        __syncthreads();
        if (col < d) {
            for (int rr = 0; rr < nr; ++rr) {
                const uint2 xv = *reinterpret_cast<const uint2*>(p.X + (int64_t)(rb + rr) * d + col);
                const float x0 = bf_lo(xv.x), x1 = bf_hi(xv.x), x2 = bf_lo(xv.y), x3 = bf_hi(xv.y);
#pragma unroll
                for (int q = 0; q < kDwExperts; ++q) {
                    const float g = s_dl[rr][q];
                    acc[q][0] += g * x0;
                    acc[q][1] += g * x1;
                    acc[q][2] += g * x2;
                    acc[q][3] += g * x3;
                }
            }
        }
    }
    if (col < d) {
        for (int q = 0; q < ne; ++q)
            *reinterpret_cast<f32x4*>(p.partial + ((int64_t)chunk * E + e0 + q) * d + col) =
                f32x4{acc[q][0], acc[q][1], acc[q][2], acc[q][3]};
    }
}

// Pass 2: dWr[e][k] = sum over chunks in ascending order.
__global__ __launch_bounds__(kThreads) void router_dw_reduce_kernel(RouterDwParams p) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t n = (int64_t)p.E * p.d;
    if (i >= n) return;
    float s = 0.0f;
    for (int c = 0; c < p.nchunks; ++c) s += p.partial[(int64_t)c * n + i];
    p.dWr[i] = s;
}

// One wave per row; Wr is staged in LDS for the router input gradient.
template <bool ROUTER>
__global__ __launch_bounds__(kThreads) void scatter_kernel(ScatterParams p, int rows_per_block) {
    extern __shared__ uint4 smem_w[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int d = p.d, K = p.K, E = p.E;
    if (ROUTER) {
        const uint4* src = reinterpret_cast<const uint4*>(p.Wr);
        for (int i = threadIdx.x; i < E * d / 8; i += kThreads) smem_w[i] = src[i];
        __syncthreads();
    }
    const uint16_t* wl = reinterpret_cast<const uint16_t*>(smem_w);
    const int rbeg = blockIdx.x * rows_per_block;
    const int rend = min(p.T, rbeg + rows_per_block);
    for (int r = rbeg + wave; r < rend; r += 4) {
        int pos[kMaxTopK];
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j)
            if (j < K) pos[j] = p.slot_of[(int64_t)r * K + j];
        for (int c0 = lane * 8; c0 < d; c0 += 512) {
            float acc[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) acc[t] = 0.0f;
#pragma unroll
            for (int j = 0; j < kMaxTopK; ++j) {
                if (j < K) {
                    float v[8];
                    unpack8(*reinterpret_cast<const uint4*>(p.dXg + (int64_t)pos[j] * d + c0), v);
#pragma unroll
                    for (int t = 0; t < 8; ++t) acc[t] += v[t];
                }
            }
            if (ROUTER) {
                for (int e = 0; e < E; ++e) {
                    const float g = p.dlogits[(int64_t)r * E + e];
                    float w[8];
                    unpack8(*reinterpret_cast<const uint4*>(wl + e * d + c0), w);
#pragma unroll
                    for (int t = 0; t < 8; ++t) acc[t] += g * w[t];
                }
            }
            *reinterpret_cast<uint4*>(p.dX + (int64_t)r * d + c0) = pack8(acc);
        }
    }
}

}  // namespace

hipError_t launch_combine(const CombineParams& p, hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    const int grid = (p.T + 3) / 4;
    if (p.silu) combine_kernel<true><<<grid, kThreads, 0, s>>>(p);
    else combine_kernel<false><<<grid, kThreads, 0, s>>>(p);
    return hipGetLastError();
}

hipError_t launch_combine_bwd(const CombineBwdParams& p, hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    const int grid = (p.T + 3) / 4;
    if (p.silu) combine_bwd_kernel<true><<<grid, kThreads, 0, s>>>(p);
    else combine_bwd_kernel<false><<<grid, kThreads, 0, s>>>(p);
    return hipGetLastError();
}

int router_dw_chunks(int T) {
    int c = (T + 127) / 128;
    return c < 1 ? 1 : (c > 256 ? 256 : c);
}

hipError_t launch_router_dw(const RouterDwParams& p, hipStream_t s) {
    dim3 grid1(p.nchunks, (p.d + 1023) / 1024, (p.E + kDwExperts - 1) / kDwExperts);
    router_dw_partial_kernel<<<grid1, kThreads, 0, s>>>(p);
    const int64_t n = (int64_t)p.E * p.d;
    router_dw_reduce_kernel<<<(unsigned)((n + kThreads - 1) / kThreads), kThreads, 0, s>>>(p);
    return hipGetLastError();
}

hipError_t launch_scatter(const ScatterParams& p, hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    const bool router = p.dlogits != nullptr && p.E > 1;
    const int rows_per_block = router ? 64 : 4;
    const int grid = (p.T + rows_per_block - 1) / rows_per_block;
    if (router)
        scatter_kernel<true><<<grid, kThreads, (size_t)p.E * p.d * 2, s>>>(p, rows_per_block);
    else
        scatter_kernel<false><<<grid, kThreads, 0, s>>>(p, rows_per_block);
    return hipGetLastError();
}

}  // namespace tmt
