// ln_row.hpp -- the LayerNorm row arithmetic (tmt-cuda/src/norm.cu:8-50),
// shared by ln_fwd_kernel (norm.hip) and the router's fused LayerNorm
// (router.hip), so that both produce the same bits.
//
// Canonical order: element k on lane (k/8) mod 64; lane sums of x and of x*x
// in ascending k from +0 (x*x of a bf16 value is exact, so the fused
// multiply-add equals multiply-then-add); xor butterfly 32..1; mean = sum/D,
// var = sumsq/D - mean^2, rstd = 1/sqrt(var + 1e-5); H = bf16(((x - mean) *
// rstd) * gamma + beta). Every other operation is rounded on its own
// (contraction off), division and sqrtf correctly rounded.
#pragma once

#include "device_util.hpp"

namespace tmt {

// Add the 8 elements of one lane piece to the lane's partial sums.
__device__ __forceinline__ void ln_accumulate(const float (&v)[8], float& ls, float& lq) {
#pragma clang fp contract(off)
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        ls = ls + v[t];
        lq = __builtin_fmaf(v[t], v[t], lq);
    }
}

// Row mean and 1/std from the lanes' partial sums (every lane gets them).
__device__ __forceinline__ void ln_finish(float ls, float lq, int d, float& mean, float& rstd) {
#pragma clang fp contract(off)
    ls += xor_lane<32>(ls);
    lq += xor_lane<32>(lq);
    ls += xor_lane<16>(ls);
    lq += xor_lane<16>(lq);
    ls += xor_lane<8>(ls);
    lq += xor_lane<8>(lq);
    ls += xor_lane<4>(ls);
    lq += xor_lane<4>(lq);
    ls += xor_lane<2>(ls);
    lq += xor_lane<2>(lq);
    ls += xor_lane<1>(ls);
    lq += xor_lane<1>(lq);
    const float D = (float)d;
    mean = ls / D;
    const float var = lq / D - mean * mean;
    rstd = 1.0f / sqrtf(var + 1e-5f);
}

// H of the 8 elements k0 .. k0 + 7 (x in v), as packed bf16.
__device__ __forceinline__ uint4 ln_apply8(const float (&v)[8], float mean, float rstd, const float* gamma,
                                           const float* beta, int k0) {
#pragma clang fp contract(off)
    const float4 g0 = *reinterpret_cast<const float4*>(gamma + k0);
    const float4 g1 = *reinterpret_cast<const float4*>(gamma + k0 + 4);
    const float4 b0 = *reinterpret_cast<const float4*>(beta + k0);
    const float4 b1 = *reinterpret_cast<const float4*>(beta + k0 + 4);
    const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const float b[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    float y[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const float xh = (v[t] - mean) * rstd;
        y[t] = xh * g[t] + b[t];
    }
    return pack8(y);
}

}  // namespace tmt
