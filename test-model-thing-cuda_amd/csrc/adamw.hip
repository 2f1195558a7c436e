// adamw.hip -- multi-tensor AdamW with global-norm clipping over the block's
// fp32 parameters and gradients (the reference's multi-tensor optimizer,
// tmt-cuda/src/adam.cu:37-96, driven by optimizer_step, model.cu:716-729).
//
// Parameters are cut once into chunks of at most kAdamChunk elements (a
// device table built at create time); every launch covers all chunks.
//
//   adamw_sumsq_kernel  per chunk: sum of grad^2 in double, in a fixed order
//                       (thread t owns the float4 groups t, t+256, ... of
//                       the chunk, x y z w in order; wave xor butterfly
//                       32..1; the four waves added in order). The last
//                       workgroup to finish (atomic ticket between
//                       device-scope fences, re-armed by that workgroup)
//                       adds the chunk sums in the same fixed order
//                       (thread t: chunks t, t+256, ...) into *sumsq. The
//                       reference adds block sums with a double atomicAdd
//                       (adam.cu:60), which is not reproducible.
//   adamw_update_kernel per element, the reference's arithmetic
//                       (adam.cu:74-85): g = grad*scale,
//                       m = b1*m + (1-b1)*g, v = b2*v + (1-b2)*g*g,
//                       w = w - lr*((m/bc1)/(sqrt(v/bc2)+eps) + wd*w),
//                       work = bf16(w); scale = min(1, clip/max(|g|_2, 1e-12))
//                       when clip > 0; a non-finite norm skips the update.
//   adamw_zero_kernel   grad = 0 (mt_zero_kernel, adam.cu:88-92).
// Every float operation is rounded on its own (no contraction), so the
// update is bit-identical to the CPU restatement.
#include "device_util.hpp"
#include "moe_internal.hpp"

#pragma clang fp contract(off)

namespace tmt {
namespace {

__device__ __forceinline__ double xor_lane_f64(double v, int off) {
    const uint64_t u = __double_as_longlong(v);
    uint32_t lo = (uint32_t)u, hi = (uint32_t)(u >> 32);
    switch (off) {
        case 32: lo = xor_lane_u32<32>(lo); hi = xor_lane_u32<32>(hi); break;
        case 16: lo = xor_lane_u32<16>(lo); hi = xor_lane_u32<16>(hi); break;
        case 8: lo = xor_lane_u32<8>(lo); hi = xor_lane_u32<8>(hi); break;
        case 4: lo = xor_lane_u32<4>(lo); hi = xor_lane_u32<4>(hi); break;
        case 2: lo = xor_lane_u32<2>(lo); hi = xor_lane_u32<2>(hi); break;
        default: lo = xor_lane_u32<1>(lo); hi = xor_lane_u32<1>(hi); break;
    }
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Sum over the workgroup in the fixed order: xor butterfly inside each wave,
// then waves 0..3 added in order. Every thread must call it.
__device__ __forceinline__ double block_sum_f64(double v, double* s_w) {
    v = v + xor_lane_f64(v, 32);
    v = v + xor_lane_f64(v, 16);
    v = v + xor_lane_f64(v, 8);
    v = v + xor_lane_f64(v, 4);
    v = v + xor_lane_f64(v, 2);
    v = v + xor_lane_f64(v, 1);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) s_w[wave] = v;
    __syncthreads();
    const double t = ((s_w[0] + s_w[1]) + s_w[2]) + s_w[3];
    __syncthreads();
    return t;
}

__global__ __launch_bounds__(kThreads) void adamw_sumsq_kernel(AdamwParams p) {
    __shared__ double s_w[4];
    __shared__ int s_last;
    const AdamwChunk c = p.chunks[blockIdx.x];
    double acc = 0.0;
    if (c.flags & kAdamwInNorm) {
        const float* g = c.grad;
        for (int i0 = threadIdx.x * 4; i0 < c.len; i0 += 4 * kThreads * 2) {
            const int i1 = i0 + 4 * kThreads;
            f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f}, b = a;
            if (i0 + 4 <= c.len) a = *reinterpret_cast<const f32x4*>(g + i0);
            else
                for (int t = 0; t < 4; ++t) a[t] = i0 + t < c.len ? g[i0 + t] : 0.f;
            if (i1 + 4 <= c.len) b = *reinterpret_cast<const f32x4*>(g + i1);
            else if (i1 < c.len)
                for (int t = 0; t < 4; ++t) b[t] = i1 + t < c.len ? g[i1 + t] : 0.f;
#pragma unroll
            for (int t = 0; t < 4; ++t) acc = acc + (double)a[t] * (double)a[t];
            if (i1 < c.len) {
#pragma unroll
                for (int t = 0; t < 4; ++t) acc = acc + (double)b[t] * (double)b[t];
            }
        }
    }
    const double tot = block_sum_f64(acc, s_w);
    if (threadIdx.x == 0) {
        p.partial[blockIdx.x] = tot;
        __threadfence();
        s_last = atomicAdd(p.ticket, 1) == (int)gridDim.x - 1;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    double s = 0.0;
    for (int k = threadIdx.x; k < p.nchunks; k += kThreads) s = s + p.partial[k];
    s = block_sum_f64(s, s_w);
    if (threadIdx.x == 0) {
        *p.sumsq = s;
        *p.ticket = 0;  // re-armed for the next step (this is the last workgroup)
    }
}

__global__ __launch_bounds__(kThreads) void adamw_update_kernel(AdamwParams p, AdamwHyper h) {
    const AdamwChunk c = p.chunks[blockIdx.x];
    if (!(c.flags & kAdamwUpdate)) return;
    const double s = *p.sumsq;
    if (!isfinite(s)) return;
    const float scale = h.clip > 0.f ? fminf(1.f, h.clip / fmaxf((float)sqrt(s), 1e-12f)) : 1.f;
    const float b1 = h.b1, b2 = h.b2, ob1 = 1.0f - h.b1, ob2 = 1.0f - h.b2;
    for (int i0 = threadIdx.x * 4; i0 < c.len; i0 += 4 * kThreads) {
        if (i0 + 4 <= c.len) {
            f32x4 g = *reinterpret_cast<const f32x4*>(c.grad + i0);
            f32x4 m = *reinterpret_cast<const f32x4*>(c.m + i0);
            f32x4 v = *reinterpret_cast<const f32x4*>(c.v + i0);
            f32x4 w = *reinterpret_cast<const f32x4*>(c.master + i0);
            float wf[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float gg = g[t] * scale;
                const float nm = b1 * m[t] + ob1 * gg;
                const float nv = b2 * v[t] + ob2 * gg * gg;
                m[t] = nm;
                v[t] = nv;
                w[t] = w[t] - h.lr * ((nm / h.bc1) / (sqrtf(nv / h.bc2) + h.eps) + h.wd * w[t]);
                wf[t] = w[t];
            }
            *reinterpret_cast<f32x4*>(c.m + i0) = m;
            *reinterpret_cast<f32x4*>(c.v + i0) = v;
            *reinterpret_cast<f32x4*>(c.master + i0) = w;
            if (c.work) {
                uint2 o;
                o.x = pack_bf2(wf[0], wf[1]);
                o.y = pack_bf2(wf[2], wf[3]);
                *reinterpret_cast<uint2*>(c.work + i0) = o;
            }
        } else {
            for (int i = i0; i < c.len; ++i) {
                const float gg = c.grad[i] * scale;
                const float nm = b1 * c.m[i] + ob1 * gg;
                const float nv = b2 * c.v[i] + ob2 * gg * gg;
                c.m[i] = nm;
                c.v[i] = nv;
                const float w = c.master[i] - h.lr * ((nm / h.bc1) / (sqrtf(nv / h.bc2) + h.eps) + h.wd * c.master[i]);
                c.master[i] = w;
                if (c.work) c.work[i] = f2bf(w);
            }
        }
    }
}

__global__ __launch_bounds__(kThreads) void adamw_zero_kernel(AdamwParams p) {
    const AdamwChunk c = p.chunks[blockIdx.x];
    for (int i0 = threadIdx.x * 4; i0 < c.len; i0 += 4 * kThreads) {
        if (i0 + 4 <= c.len) *reinterpret_cast<f32x4*>(c.grad + i0) = f32x4{0.f, 0.f, 0.f, 0.f};
        else
            for (int i = i0; i < c.len; ++i) c.grad[i] = 0.f;
    }
}

}  // namespace

hipError_t launch_adamw_sumsq(const AdamwParams& p, hipStream_t s) {
    if (p.nchunks <= 0) return hipSuccess;
    adamw_sumsq_kernel<<<p.nchunks, kThreads, 0, s>>>(p);
    return hipGetLastError();
}

hipError_t launch_adamw_update(const AdamwParams& p, const AdamwHyper& h, hipStream_t s) {
    if (p.nchunks <= 0) return hipSuccess;
    adamw_update_kernel<<<p.nchunks, kThreads, 0, s>>>(p, h);
    return hipGetLastError();
}

hipError_t launch_adamw_zero(const AdamwParams& p, hipStream_t s) {
    if (p.nchunks <= 0) return hipSuccess;
    adamw_zero_kernel<<<p.nchunks, kThreads, 0, s>>>(p);
    return hipGetLastError();
}

}  // namespace tmt
