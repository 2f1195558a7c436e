// norm.hip -- the LayerNorm that precedes the MoE block in TMT, as part of
// the block (tmt-cuda/src/norm.cu:8-106; caller tmt-cuda/src/model.cu:509-514,
// 678-680).
//
//   ln_fwd      H = bf16(((x - mean) * rstd) * gamma + beta), one wave per row,
//               in the canonical order of ln_row.hpp, which the CPU oracle
//               restates (the reference's block tree and rsqrtf are not
//               reproducible, this order is). H is therefore bit-identical to
//               the oracle's, and so are the router logits computed from it.
//               For routed batches the router computes the same rows itself
//               (router.hip) and this kernel is not launched.
//   ln_bwd_rows dS = rstd * ((g - mean(g)) - xh * mean(g * xh)) with g = dH * gamma,
//               xh = (x - mean) * rstd, one wave per row.
//   ln_dgb      dgamma = sum_r dH * xh, dbeta = sum_r dH: chunk partials over
//               512-row chunks (rows ascending, waves added in order), then a
//               fixed-order sum over chunks (colsum) -- no atomics (the
//               reference uses atomicAdd, norm.cu:68-69).
// For d <= kLnFusedMaxD the backward rows and the chunk partials run inside
// the dX scatter instead (pointwise.hip) and only colsum runs from here; the
// two kernels above are the path for wider rows.
#include "device_util.hpp"
#include "ln_row.hpp"
#include "moe_internal.hpp"

// Every float operation below is rounded on its own: no contraction into
// fused multiply-adds except the explicit one in ln_row.hpp. Division and
// sqrtf are correctly rounded (hipcc's default for fp32).
#pragma clang fp contract(off)

namespace tmt {
namespace {

__device__ __forceinline__ void row_stats(const uint16_t* x, int d, int lane, float& mean, float& rstd) {
    float ls = 0.0f, lq = 0.0f;
    for (int k0 = lane * 8; k0 < d; k0 += 512) {
        float v[8];
        unpack8(*reinterpret_cast<const uint4*>(x + k0), v);
        ln_accumulate(v, ls, lq);
    }
    ln_finish(ls, lq, d, mean, rstd);
}

__global__ __launch_bounds__(kThreads) void ln_fwd_kernel(LayerNormParams p) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= p.T) return;
    const int d = p.d;
    const uint16_t* x = p.S + (int64_t)r * d;
    float mean, rstd;
    row_stats(x, d, lane, mean, rstd);
    for (int k0 = lane * 8; k0 < d; k0 += 512) {
        float v[8];
        unpack8(*reinterpret_cast<const uint4*>(x + k0), v);
        *reinterpret_cast<uint4*>(p.H + (int64_t)r * d + k0) = ln_apply8(v, mean, rstd, p.gamma, p.beta, k0);
    }
    if (lane == 0) {
        p.mean[r] = mean;
        p.rstd[r] = rstd;
    }
}

__global__ __launch_bounds__(kThreads) void ln_bwd_rows_kernel(LayerNormParams p) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= p.T) return;
    const int d = p.d;
    const uint16_t* x = p.S + (int64_t)r * d;
    const uint16_t* dh = p.dH + (int64_t)r * d;
    const float mean = p.mean[r], rstd = p.rstd[r];
    float s1 = 0.0f, s2 = 0.0f;
    for (int k0 = lane * 8; k0 < d; k0 += 512) {
        float v[8], gy[8];
        unpack8(*reinterpret_cast<const uint4*>(x + k0), v);
        unpack8(*reinterpret_cast<const uint4*>(dh + k0), gy);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float g = gy[t] * p.gamma[k0 + t];
            const float xh = (v[t] - mean) * rstd;
            s1 = s1 + g;
            s2 = s2 + g * xh;
        }
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    const float a = s1 / (float)d, b = s2 / (float)d;
    for (int k0 = lane * 8; k0 < d; k0 += 512) {
        float v[8], gy[8], out[8];
        unpack8(*reinterpret_cast<const uint4*>(x + k0), v);
        unpack8(*reinterpret_cast<const uint4*>(dh + k0), gy);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float g = gy[t] * p.gamma[k0 + t];
            const float xh = (v[t] - mean) * rstd;
            out[t] = rstd * ((g - a) - xh * b);
        }
        *reinterpret_cast<uint4*>(p.dS + (int64_t)r * d + k0) = pack8(out);
    }
}

// Pass 1: block (chunk of kLnRows rows, 256 columns); lane l of every wave
// owns columns 4l..4l+3, wave w rows w, w+4, ... of the chunk (ascending).
constexpr int kLnRows = 512;
constexpr int kLnCols = 256;
__global__ __launch_bounds__(kThreads) void ln_dgb_partial_kernel(LayerNormParams p) {
    __shared__ f32x4 s_part[3][2][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int chunk = blockIdx.x;
    const int col = blockIdx.y * kLnCols + lane * 4;
    const int d = p.d;
    const int r0 = chunk * kLnRows, r1 = min(p.T, r0 + kLnRows);
    const bool cok = col < d;
    const int ccol = cok ? col : 0;
    f32x4 ag = f32x4{0.f, 0.f, 0.f, 0.f}, ab = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int rb = r0 + wave; rb < r1; rb += 16) {
        uint2 xv[4], gv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = min(rb + 4 * u, r1 - 1);
            xv[u] = *reinterpret_cast<const uint2*>(p.S + (int64_t)r * d + ccol);
            gv[u] = *reinterpret_cast<const uint2*>(p.dH + (int64_t)r * d + ccol);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = rb + 4 * u;
            if (r >= r1) break;  // wave-uniform
            const float mean = p.mean[r], rstd = p.rstd[r];
            const float x[4] = {bf_lo(xv[u].x), bf_hi(xv[u].x), bf_lo(xv[u].y), bf_hi(xv[u].y)};
            const float g[4] = {bf_lo(gv[u].x), bf_hi(gv[u].x), bf_lo(gv[u].y), bf_hi(gv[u].y)};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float xh = (x[t] - mean) * rstd;
                ag[t] = ag[t] + g[t] * xh;
                ab[t] = ab[t] + g[t];
            }
        }
    }
    if (wave > 0) {
        s_part[wave - 1][0][lane] = ag;
        s_part[wave - 1][1][lane] = ab;
    }
    __syncthreads();
    if (wave == 0 && cok) {
        for (int w = 0; w < 3; ++w) {
            ag += s_part[w][0][lane];
            ab += s_part[w][1][lane];
        }
        *reinterpret_cast<f32x4*>(p.partial + ((int64_t)chunk * 2) * d + col) = ag;
        *reinterpret_cast<f32x4*>(p.partial + ((int64_t)chunk * 2 + 1) * d + col) = ab;
    }
}

// Fixed-order column sums of a [nrows][ncols] fp32 matrix (ncols a multiple
// of 4), in two levels: level 1 sums groups of kColGroup consecutive rows
// (wave w takes rows w*16 .. w*16+15 of the group in ascending order, the
// four waves are then added in order), level 2 adds the group sums in
// ascending order. Columns [0, split) go to out_lo, the rest to out_hi.
constexpr int kColGroup = 64;
__global__ __launch_bounds__(kThreads) void colsum_level1_kernel(const float* in, int nrows, int ncols,
                                                                 float* out) {
    __shared__ f32x4 s_part[3][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = blockIdx.x * 256 + lane * 4;
    const int g = blockIdx.y;
    const bool cok = col < ncols;
    const int r0 = g * kColGroup + wave * 16;
    const int n = max(0, min(16, nrows - r0));
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    if (cok && n > 0) {
        f32x4 v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i)
            v[i] = *reinterpret_cast<const f32x4*>(in + (int64_t)(r0 + min(i, n - 1)) * ncols + col);
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (i < n) acc += v[i];
    }
    if (wave > 0) s_part[wave - 1][lane] = acc;
    __syncthreads();
    if (wave == 0 && cok) {
        acc += s_part[0][lane];
        acc += s_part[1][lane];
        acc += s_part[2][lane];
        *reinterpret_cast<f32x4*>(out + (int64_t)g * ncols + col) = acc;
    }
}

__global__ __launch_bounds__(kThreads) void colsum_level2_kernel(const float* in, int ngroups, int ncols,
                                                                 int split, float* out_lo, float* out_hi) {
    const int col = (blockIdx.x * kThreads + threadIdx.x) * 4;
    if (col >= ncols) return;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int g0 = 0; g0 < ngroups; g0 += 8) {
        f32x4 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v[i] = *reinterpret_cast<const f32x4*>(in + (int64_t)min(g0 + i, ngroups - 1) * ncols + col);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (g0 + i < ngroups) acc += v[i];
    }
    float* dst = col < split ? out_lo + col : out_hi + (col - split);
    *reinterpret_cast<f32x4*>(dst) = acc;
}

}  // namespace

int ln_chunks(int T) {
    const int c = (T + kLnRows - 1) / kLnRows;
    return c < 1 ? 1 : c;
}

int colsum_groups(int nrows) {
    const int g = (nrows + kColGroup - 1) / kColGroup;
    return g < 1 ? 1 : g;
}

hipError_t launch_colsum(const float* in, int nrows, int ncols, float* scratch, int split, float* out_lo,
                         float* out_hi, hipStream_t s) {
    if (ncols % 4 != 0) return hipErrorInvalidValue;
    const int ng = colsum_groups(nrows);
    colsum_level1_kernel<<<dim3((ncols + 255) / 256, ng), kThreads, 0, s>>>(in, nrows, ncols, scratch);
    colsum_level2_kernel<<<(ncols / 4 + kThreads - 1) / kThreads, kThreads, 0, s>>>(scratch, ng, ncols, split,
                                                                                   out_lo, out_hi);
    return hipGetLastError();
}

hipError_t launch_ln_fwd(const LayerNormParams& p, hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    ln_fwd_kernel<<<(p.T + 3) / 4, kThreads, 0, s>>>(p);
    return hipGetLastError();
}

hipError_t launch_ln_bwd(const LayerNormParams& p, hipStream_t s) {
    if (p.T > 0) ln_bwd_rows_kernel<<<(p.T + 3) / 4, kThreads, 0, s>>>(p);
    const int nch = ln_chunks(p.T);
    ln_dgb_partial_kernel<<<dim3(nch, (p.d + kLnCols - 1) / kLnCols), kThreads, 0, s>>>(p);
    return launch_colsum(p.partial, nch, 2 * p.d, p.partial2, p.d, p.dgamma, p.dbeta, s);
}

}  // namespace tmt
