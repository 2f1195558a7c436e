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
//                       32..1; the four waves added in order).
//   adamw_norm_kernel   one workgroup of 1024 threads adds the chunk sums in
//                       the same kind of fixed order (thread t: chunks t,
//                       t+1024, ...; butterfly; sixteen waves in order) into
//                       *sumsq. The reference adds block sums with a double
//                       atomicAdd (adam.cu:60), which is not reproducible; a
//                       last-workgroup ticket instead of this second launch
//                       needs a device-scope fence per workgroup, i.e. an L2
//                       write-back per chunk (measured 7x slower).
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
// then the NW waves added in order. Every thread must call it.
template <int NW>
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
    double t = s_w[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) t = t + s_w[w];
    __syncthreads();
    return t;
}

__global__ __launch_bounds__(kThreads) void adamw_sumsq_kernel(AdamwParams p) {
    __shared__ double s_w[4];
    const AdamwChunk c = p.chunks[blockIdx.x];
    double acc = 0.0;
    if ((c.flags & kAdamwInNorm) && c.len == kAdamChunk) {
        // Full chunk: all eight of the thread's groups in flight at once.
        constexpr int G = kAdamChunk / (4 * kThreads);
        f32x4 a[G];
#pragma unroll
        for (int u = 0; u < G; ++u)
            a[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(c.grad) + threadIdx.x + u * kThreads);
#pragma unroll
        for (int u = 0; u < G; ++u)
#pragma unroll
            for (int t = 0; t < 4; ++t) acc = acc + (double)a[u][t] * (double)a[u][t];
    } else if (c.flags & kAdamwInNorm) {
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
    const double tot = block_sum_f64<4>(acc, s_w);
    if (threadIdx.x == 0) p.partial[blockIdx.x] = tot;
}

constexpr int kNormThreads = 1024;
__global__ __launch_bounds__(kNormThreads) void adamw_norm_kernel(AdamwParams p) {
    __shared__ double s_w[kNormThreads / 64];
    double s = 0.0;
    for (int k0 = threadIdx.x; k0 < p.nchunks; k0 += 8 * kNormThreads) {
        double v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int k = k0 + u * kNormThreads;
            v[u] = k < p.nchunks ? p.partial[k] : 0.0;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (k0 + u * kNormThreads < p.nchunks) s = s + v[u];
    }
    s = block_sum_f64<kNormThreads / 64>(s, s_w);
    if (threadIdx.x == 0) *p.sumsq = s;
}

// One element of the update (adam.cu:78-84); w, m, v in place.
__device__ __forceinline__ void adam_elem(float g, float& m, float& v, float& w, float scale,
                                          const AdamwHyper& h, float ob1, float ob2) {
    const float gg = g * scale;
    const float nm = h.b1 * m + ob1 * gg;
    const float nv = h.b2 * v + ob2 * gg * gg;
    m = nm;
    v = nv;
    w = w - h.lr * ((nm / h.bc1) / (sqrtf(nv / h.bc2) + h.eps) + h.wd * w);
}

__global__ __launch_bounds__(kThreads) void adamw_update_kernel(AdamwParams p, AdamwHyper h) {
    const AdamwChunk c = p.chunks[blockIdx.x];
    if (!(c.flags & kAdamwUpdate)) return;
    const double s = *p.sumsq;
    if (!isfinite(s)) return;
    const float scale = h.clip > 0.f ? fminf(1.f, h.clip / fmaxf((float)sqrt(s), 1e-12f)) : 1.f;
    const float ob1 = 1.0f - h.b1, ob2 = 1.0f - h.b2;
    const f32x4* __restrict__ gp = reinterpret_cast<const f32x4*>(c.grad);
    f32x4* __restrict__ mp = reinterpret_cast<f32x4*>(c.m);
    f32x4* __restrict__ vp = reinterpret_cast<f32x4*>(c.v);
    f32x4* __restrict__ wp = reinterpret_cast<f32x4*>(c.master);
    uint2* __restrict__ op = reinterpret_cast<uint2*>(c.work);
    const int nvec = c.len / 4;
    // Two 4-element groups per thread and iteration, all eight loads first.
    for (int j0 = threadIdx.x; j0 < nvec; j0 += 2 * kThreads) {
        const int j1 = j0 + kThreads;
        const bool two = j1 < nvec;
        f32x4 g[2], m[2], v[2], w[2];
        g[0] = __builtin_nontemporal_load(gp + j0);
        m[0] = mp[j0];
        v[0] = vp[j0];
        w[0] = wp[j0];
        if (two) {
            g[1] = __builtin_nontemporal_load(gp + j1);
            m[1] = mp[j1];
            v[1] = vp[j1];
            w[1] = wp[j1];
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (u == 1 && !two) break;
            const int j = u == 0 ? j0 : j1;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                float mm = m[u][t], vv = v[u][t], ww = w[u][t];
                adam_elem(g[u][t], mm, vv, ww, scale, h, ob1, ob2);
                m[u][t] = mm;
                v[u][t] = vv;
                w[u][t] = ww;
            }
            mp[j] = m[u];
            vp[j] = v[u];
            wp[j] = w[u];
            if (op) {
                uint2 o;
                o.x = pack_bf2(w[u][0], w[u][1]);
                o.y = pack_bf2(w[u][2], w[u][3]);
                op[j] = o;
            }
        }
    }
    // Tail of a parameter whose size is not a multiple of 4.
    for (int i = nvec * 4 + threadIdx.x; i < c.len; i += kThreads) {
        float mm = c.m[i], vv = c.v[i], ww = c.master[i];
        adam_elem(c.grad[i], mm, vv, ww, scale, h, ob1, ob2);
        c.m[i] = mm;
        c.v[i] = vv;
        c.master[i] = ww;
        if (c.work) c.work[i] = f2bf(ww);
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
    adamw_norm_kernel<<<1, kNormThreads, 0, s>>>(p);
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
