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
// two kernels above are the path for wider rows and for widths that are not
// a multiple of 64. Any d >= 1 is accepted: rows whose width or strides are
// not multiples of 8 elements are read and written element by element, with
// the same summation order (missing elements of the last 8-element piece
// count as zeros, which leave every sum unchanged).
#include "device_util.hpp"
#include "ln_row.hpp"
#include "moe_internal.hpp"

// Every float operation below is rounded on its own: no contraction into
// fused multiply-adds except the explicit one in ln_row.hpp. Division and
// sqrtf are correctly rounded (hipcc's default for fp32).
#pragma clang fp contract(off)

namespace tmt {
namespace {

// The 8 elements k0 .. k0 + 7 of a row: one 16-byte load when VEC (d, the
// row strides and the base pointers are multiples of 8 elements / 16 bytes),
// else element by element, with zeros from column d on. Zeros leave the row
// sums unchanged (x + 0 = x, fma(0, 0, s) = s), so both forms give the same
// statistics.
template <bool VEC>
__device__ __forceinline__ void load_row8(const uint16_t* row, int k0, int d, float (&v)[8]) {
    if constexpr (VEC) {
        unpack8(*reinterpret_cast<const uint4*>(row + k0), v);
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) v[t] = k0 + t < d ? bf1(row[k0 + t]) : 0.0f;
    }
}

template <bool VEC>
__device__ __forceinline__ void row_stats(const uint16_t* x, int d, int lane, float& mean, float& rstd) {
    float ls = 0.0f, lq = 0.0f;
    for (int k0 = lane * 8; k0 < d; k0 += 512) {
        float v[8];
        load_row8<VEC>(x, k0, d, v);
        ln_accumulate(v, ls, lq);
    }
    ln_finish(ls, lq, d, mean, rstd);
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void ln_fwd_kernel(LayerNormParams p) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= p.T) return;
    const int d = p.d;
    const uint16_t* x = p.S + (int64_t)r * p.lds;
    uint16_t* hrow = p.H + (int64_t)r * p.ldh;
    float mean, rstd;
    row_stats<VEC>(x, d, lane, mean, rstd);
    for (int k0 = lane * 8; k0 < p.ldh; k0 += 512) {
        if constexpr (VEC) {
            uint4 hv = make_uint4(0, 0, 0, 0);  // columns [d, ldh): zeros
            if (k0 < d) {
                float v[8];
                unpack8(*reinterpret_cast<const uint4*>(x + k0), v);
                hv = ln_apply8(v, mean, rstd, p.gamma, p.beta, k0);
            }
            *reinterpret_cast<uint4*>(hrow + k0) = hv;
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int k = k0 + t;
                if (k >= p.ldh) break;
                uint16_t hv = 0;
                if (k < d) {
                    const float xh = (bf1(x[k]) - mean) * rstd;
                    hv = f2bf(xh * p.gamma[k] + p.beta[k]);
                }
                hrow[k] = hv;
            }
        }
    }
    if (lane == 0) {
        p.mean[r] = mean;
        p.rstd[r] = rstd;
    }
}

// Rows of at most NP * 512 elements (16-byte pieces): each lane loads its
// pieces once into registers, so the normalisation does not read the row a
// second time after the statistics (one memory round trip per row instead
// of two). The sums run over the same pieces in the same order as
// row_stats, so mean, 1/std and H are bit-identical to ln_fwd_kernel<true>.
template <int NP>
__global__ __launch_bounds__(kThreads) void ln_fwd_reg_kernel(LayerNormParams p) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= p.T) return;
    const int d = p.d;
    const uint16_t* x = p.S + (int64_t)r * p.lds;
    uint16_t* hrow = p.H + (int64_t)r * p.ldh;
    uint4 raw[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const int k0 = lane * 8 + 512 * i;
        raw[i] = k0 < d ? *reinterpret_cast<const uint4*>(x + k0) : make_uint4(0, 0, 0, 0);
    }
    float ls = 0.0f, lq = 0.0f;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        if (lane * 8 + 512 * i < d) {
            float v[8];
            unpack8(raw[i], v);
            ln_accumulate(v, ls, lq);
        }
    }
    float mean, rstd;
    ln_finish(ls, lq, d, mean, rstd);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const int k0 = lane * 8 + 512 * i;
        if (k0 >= p.ldh) break;
        uint4 hv = make_uint4(0, 0, 0, 0);  // columns [d, ldh): zeros
        if (k0 < d) {
            float v[8];
            unpack8(raw[i], v);
            hv = ln_apply8(v, mean, rstd, p.gamma, p.beta, k0);
        }
        *reinterpret_cast<uint4*>(hrow + k0) = hv;
    }
    if (lane == 0) {
        p.mean[r] = mean;
        p.rstd[r] = rstd;
    }
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void ln_bwd_rows_kernel(LayerNormParams p) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= p.T) return;
    const int d = p.d;
    const uint16_t* x = p.S + (int64_t)r * p.lds;
    const uint16_t* dh = p.dH + (int64_t)r * p.ldh;
    const float mean = p.mean[r], rstd = p.rstd[r];
    float s1 = 0.0f, s2 = 0.0f;
    for (int k0 = lane * 8; k0 < d; k0 += 512) {
        float v[8], gy[8];
        load_row8<VEC>(x, k0, d, v);
        load_row8<VEC>(dh, k0, d, gy);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            if (!VEC && k0 + t >= d) break;
            const float g = gy[t] * p.gamma[k0 + t];
            const float xh = (v[t] - mean) * rstd;
            s1 = s1 + g;
            s2 = s2 + g * xh;
        }
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    const float a = s1 / (float)d, b = s2 / (float)d;
    uint16_t* ds = p.dS + (int64_t)r * p.lds;
    for (int k0 = lane * 8; k0 < d; k0 += 512) {
        float v[8], gy[8], out[8];
        load_row8<VEC>(x, k0, d, v);
        load_row8<VEC>(dh, k0, d, gy);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float g = (VEC || k0 + t < d) ? gy[t] * p.gamma[k0 + t] : 0.0f;
            const float xh = (v[t] - mean) * rstd;
            out[t] = rstd * ((g - a) - xh * b);
        }
        if constexpr (VEC) {
            *reinterpret_cast<uint4*>(ds + k0) = pack8(out);
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t)
                if (k0 + t < d) ds[k0 + t] = f2bf(out[t]);
        }
    }
}

// Pass 1: block (chunk of kLnRows rows, 256 columns); lane l of every wave
// owns columns 4l..4l+3, wave w rows w, w+4, ... of the chunk (ascending).
constexpr int kLnRows = 512;
constexpr int kLnCols = 256;
// Partials are rows of ln_width4(d) floats; columns [d, ln_width4(d)) hold zeros.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void ln_dgb_partial_kernel(LayerNormParams p) {
    __shared__ f32x4 s_part[3][2][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int chunk = blockIdx.x;
    const int col = blockIdx.y * kLnCols + lane * 4;
    const int d = p.d, pw = ln_width4(d);
    const int r0 = chunk * kLnRows, r1 = min(p.T, r0 + kLnRows);
    const bool cok = col < d;
    const int ccol = cok ? col : 0;
    // four columns of row r of a bf16 matrix with row stride ld (zeros from column d on)
    auto load4 = [&](const uint16_t* base, int ld, int r, float (&v)[4]) {
        const uint16_t* q = base + (int64_t)r * ld + ccol;
        if constexpr (VEC) {
            const uint2 w = *reinterpret_cast<const uint2*>(q);
            v[0] = bf_lo(w.x); v[1] = bf_hi(w.x); v[2] = bf_lo(w.y); v[3] = bf_hi(w.y);
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) v[t] = ccol + t < d ? bf1(q[t]) : 0.0f;
        }
    };
    f32x4 ag = f32x4{0.f, 0.f, 0.f, 0.f}, ab = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int rb = r0 + wave; rb < r1; rb += 16) {
        float xv[4][4], gv[4][4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = min(rb + 4 * u, r1 - 1);
            load4(p.S, p.lds, r, xv[u]);
            load4(p.dH, p.ldh, r, gv[u]);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = rb + 4 * u;
            if (r >= r1) break;  // wave-uniform
            const float mean = p.mean[r], rstd = p.rstd[r];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float xh = (xv[u][t] - mean) * rstd;
                ag[t] = ag[t] + gv[u][t] * xh;
                ab[t] = ab[t] + gv[u][t];
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
        *reinterpret_cast<f32x4*>(p.partial + ((int64_t)chunk * 2) * pw + col) = ag;
        *reinterpret_cast<f32x4*>(p.partial + ((int64_t)chunk * 2 + 1) * pw + col) = ab;
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
                                                                 int split, int width, float* out_lo,
                                                                 float* out_hi) {
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
    const int c = col < split ? col : col - split;
    float* dst = (col < split ? out_lo : out_hi) + c;
    if (c + 4 <= width) {
        *reinterpret_cast<f32x4*>(dst) = acc;
    } else {
        for (int t = 0; t < 4 && c + t < width; ++t) dst[t] = acc[t];
    }
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

hipError_t launch_colsum(const float* in, int nrows, int ncols, float* scratch, int split, int width,
                         float* out_lo, float* out_hi, hipStream_t s) {
    if (ncols % 4 != 0 || split % 4 != 0 || width > split || width > ncols - split) return hipErrorInvalidValue;
    const int ng = colsum_groups(nrows);
    colsum_level1_kernel<<<dim3((ncols + 255) / 256, ng), kThreads, 0, s>>>(in, nrows, ncols, scratch);
    colsum_level2_kernel<<<(ncols / 4 + kThreads - 1) / kThreads, kThreads, 0, s>>>(scratch, ng, ncols, split,
                                                                                   width, out_lo, out_hi);
    return hipGetLastError();
}

namespace {
bool al16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }
// 16-byte row accesses when d and both row strides are multiples of 8
// elements and every row base is 16-byte aligned; element accesses otherwise.
bool ln_vec(const LayerNormParams& p, bool fwd) {
    if (p.d % 8 != 0 || p.lds % 8 != 0 || p.ldh % 8 != 0 || !al16(p.S)) return false;
    return fwd ? al16(p.H) : (al16(p.dH) && al16(p.dS));
}
}  // namespace

hipError_t launch_ln_fwd(const LayerNormParams& p, hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    if (p.d < 1 || p.lds < p.d || p.ldh < p.d) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)((p.T + 3) / 4);
    if (!ln_vec(p, true)) {
        ln_fwd_kernel<false><<<grid, kThreads, 0, s>>>(p);
    } else {
        switch ((p.ldh + 511) / 512) {  // 16-byte pieces per lane, H's padded columns included
            case 1: ln_fwd_reg_kernel<1><<<grid, kThreads, 0, s>>>(p); break;
            case 2: ln_fwd_reg_kernel<2><<<grid, kThreads, 0, s>>>(p); break;
            case 3: ln_fwd_reg_kernel<3><<<grid, kThreads, 0, s>>>(p); break;
            case 4: ln_fwd_reg_kernel<4><<<grid, kThreads, 0, s>>>(p); break;
            default: ln_fwd_kernel<true><<<grid, kThreads, 0, s>>>(p); break;
        }
    }
    return hipGetLastError();
}

hipError_t launch_ln_bwd(const LayerNormParams& p, hipStream_t s) {
    if (p.d < 1 || p.lds < p.d || p.ldh < p.d) return hipErrorInvalidValue;
    const bool vec = ln_vec(p, false);
    const int nch = ln_chunks(p.T), pw = ln_width4(p.d);
    const dim3 grid(nch, (p.d + kLnCols - 1) / kLnCols);
    if (vec) {
        if (p.T > 0) ln_bwd_rows_kernel<true><<<(p.T + 3) / 4, kThreads, 0, s>>>(p);
        ln_dgb_partial_kernel<true><<<grid, kThreads, 0, s>>>(p);
    } else {
        if (p.T > 0) ln_bwd_rows_kernel<false><<<(p.T + 3) / 4, kThreads, 0, s>>>(p);
        ln_dgb_partial_kernel<false><<<grid, kThreads, 0, s>>>(p);
    }
    return launch_colsum(p.partial, nch, 2 * pw, p.partial2, pw, p.d, p.dgamma, p.dbeta, s);
}

}  // namespace tmt
