// device_util.hpp -- small gfx950 device helpers shared by the kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tmt {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// bf16 bit patterns packed two per dword: element 2i in the low half.
__device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }
__device__ __forceinline__ float bf1(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }

// Round-to-nearest-even fp32 -> bf16 (the conversion instruction of gfx950).
__device__ __forceinline__ uint16_t f2bf(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}
// Two values in one v_cvt_pk_bf16_f32 (the same rounding as f2bf on each;
// converting them one at a time costs two conversions, a shift and an or).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// One wave-wide 16-byte-per-lane load from global memory into LDS at
// lds_base + 16 * lane (lds_base wave-uniform); M0 is declared clobbered.
// These loads count on the vector-memory counter like any other, but the
// compiler does not see them: a compiler-placed wait for a later load waits
// for them too (the counter completes in order).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16_lds(const void* g, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_base) : "m0", "memory");
}
// The same with 4 bytes per lane (to lds_base + 4 * lane).
__device__ __forceinline__ void dma4_lds(const void* g, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds_base) : "m0", "memory");
}
#pragma clang diagnostic pop
// LDS address of a pointer into shared memory.
__device__ __forceinline__ uint32_t lds_u32(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// The M tiles (TBM slots each) of the experts' slot segments, one expert per
// lane (E <= 64): lane e holds expert e's first tile and first slot, so a
// tile's expert is one ballot rather than a walk over the offsets. Built
// once per workgroup (one vector load of the offsets and a wave prefix sum);
// two VGPRs stay live.
struct ExpertTiles {
    int first, beg;   // per lane: first tile and first slot of expert `lane` (lanes >= E: total, end)
    int total, end;   // wave-uniform: tiles of all experts, offsets[E]
};
template <int TBM>
__device__ __forceinline__ ExpertTiles expert_tiles(const int32_t* offsets, int E, int lane) {
    ExpertTiles m;
    m.end = __builtin_amdgcn_readfirstlane(offsets[E]);
    m.beg = lane < E ? offsets[lane] : m.end;
    const int nxt = __shfl_down(m.beg, 1);
    const int tiles = lane < E ? ((lane + 1 < E ? nxt : m.end) - m.beg + TBM - 1) / TBM : 0;
    int incl = tiles;  // inclusive prefix over the lanes
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o);
        if (lane >= o) incl += v;
    }
    m.first = incl - tiles;
    m.total = __builtin_amdgcn_readlane(incl, 63);
    return m;
}
// Expert segment of M tile mt (wave-uniform): expert, first slot, rows;
// false when mt is past the last tile.
template <int TBM>
__device__ __forceinline__ bool expert_tile(const ExpertTiles& m, int mt, int& e, int& row0, int& rows) {
    const int lane = __lane_id();
    const int dn = __shfl_down(m.first, 1);
    const int next = lane == 63 ? m.total : dn;  // first tile of the next expert
    const uint64_t hit = __ballot(m.first <= mt && mt < next);
    if (hit == 0) return false;
    e = __builtin_ctzll(hit);
    row0 = __builtin_amdgcn_readlane(m.beg, e) + (mt - __builtin_amdgcn_readlane(m.first, e)) * TBM;
    const int end = e < 63 ? __builtin_amdgcn_readlane(m.beg, e + 1) : m.end;
    rows = min(TBM, end - row0);
    return true;
}

// Unpack 8 bf16 held in a uint4 into fp32.
__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
    f[0] = bf_lo(v.x); f[1] = bf_hi(v.x);
    f[2] = bf_lo(v.y); f[3] = bf_hi(v.y);
    f[4] = bf_lo(v.z); f[5] = bf_hi(v.z);
    f[6] = bf_lo(v.w); f[7] = bf_hi(v.w);
}
__device__ __forceinline__ uint4 pack8(const float* f) {
    uint4 v;
    v.x = pack_bf2(f[0], f[1]);
    v.y = pack_bf2(f[2], f[3]);
    v.z = pack_bf2(f[4], f[5]);
    v.w = pack_bf2(f[6], f[7]);
    return v;
}

// SiLU and its derivative (reference tmt-cuda/src/common.h:15-24) with the
// hardware exp2 / reciprocal: x * sigmoid(x), g*s*(1 + x(1 - s)).
__device__ __forceinline__ float sigmoid_fast(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}
__device__ __forceinline__ float silu_fast(float x) { return x * sigmoid_fast(x); }
__device__ __forceinline__ float dsilu_fast(float x) {
    float s = sigmoid_fast(x);
    return s * (1.0f + x * (1.0f - s));
}
// Both from one sigmoid: the up GEMM's epilogue writes SiLU(U) for the down
// GEMM and silu'(U) for the backward (GEMM_DACT multiplies by it), so the
// exp / reciprocal pair runs once per element of U, in the forward.
// silu'(x) = s(1 + x(1 - s)) = s + a(1 - s) with a = x s: one subtraction and
// one fused multiply-add (the up GEMM's epilogue is bound by these VALU
// instructions).
__device__ __forceinline__ void silu_dsilu(float x, float& a, float& da) {
    const float s = sigmoid_fast(x);
    a = x * s;
    da = __builtin_fmaf(a, 1.0f - s, s);
}

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63); }

// Value of lane (lane ^ OFF), moved by VALU cross-lane operations instead of
// the LDS permute unit: DPP quad permutes / row rotate / half-row mirror for
// OFF <= 8, and the gfx950 row-swap instructions for 16 and 32
// (permlane16_swap(v, v) yields rows {0,0,2,2} and {1,1,3,3};
// permlane32_swap(v, v) yields halves {lo,lo} and {hi,hi}).
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
template <int C>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, C, 0xF, 0xF, false);
}
template <int OFF>
__device__ __forceinline__ uint32_t xor_lane_u32(uint32_t v) {
    static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8 || OFF == 16 || OFF == 32, "xor offset");
    if constexpr (OFF == 1) return dpp_mov<0xB1>(v);                  // quad_perm [1,0,3,2]
    else if constexpr (OFF == 2) return dpp_mov<0x4E>(v);             // quad_perm [2,3,0,1]
    else if constexpr (OFF == 4) return dpp_mov<0x1B>(dpp_mov<0x141>(v));  // half mirror, quad [3,2,1,0]
    else if constexpr (OFF == 8) return dpp_mov<0x128>(v);            // row_ror:8
    else if constexpr (OFF == 16) {
        const u32x2_t s = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (threadIdx.x & 16) ? s[0] : s[1];
    } else {
        const u32x2_t s = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (threadIdx.x & 32) ? s[0] : s[1];
    }
}
template <int OFF>
__device__ __forceinline__ float xor_lane(float v) {
    return __uint_as_float(xor_lane_u32<OFF>(__float_as_uint(v)));
}
template <int OFF>
__device__ __forceinline__ int xor_lane(int v) {
    return (int)xor_lane_u32<OFF>((uint32_t)v);
}

__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }
__device__ __forceinline__ int shfl_xor(int v, int m) { return __shfl_xor(v, m, 64); }

// Full-wave xor butterfly sum with offsets 32,16,...,1: every lane ends with
// the same value (each step adds two equal-shaped partial trees).
__device__ __forceinline__ float wave_sum(float v) {
    v = v + xor_lane<32>(v);
    v = v + xor_lane<16>(v);
    v = v + xor_lane<8>(v);
    v = v + xor_lane<4>(v);
    v = v + xor_lane<2>(v);
    v = v + xor_lane<1>(v);
    return v;
}

}  // namespace tmt
