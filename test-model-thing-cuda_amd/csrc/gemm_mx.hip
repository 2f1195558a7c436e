// gemm_mx.hip -- MXFP4 expert GEMMs on gfx950's scaled MFMA.
//
// The MXFP4 forward (no counterpart in the reference, which has no FP4
// path) with activations in MX form as well, so both operands feed
// v_mfma_scale_f32_32x32x64_f8f6f4 directly:
//   weights      e2m1 codes + e8m0 scales per 32 along K (the layout of
//                tmt_moe_forward_mxfp4: codes [N][K/2], low nibble first;
//                scales [K/32][N]);
//   activations  the sum of two e2m3 (FP6) terms, each with its own e8m0
//                scale per 32 along K: x ~ q0 * 2^(s0-127) + q1 * 2^(s1-127),
//                q0 = RNE(x / 2^e0) with e0 = floor(log2 max|x|) - 2 over the
//                block, q1 the same rounding of the residual x - q0 * 2^e0.
//                Relative L2 error about 4e-4 on the c5 operands, against
//                3e-2 for one term.
// FP6 x FP4 products issue at the 8-pass rate, so the two terms together take
// half the MFMA time of one bf16 product over the same K.
//
// Activation tensors ("MX6x2"), rows R, length K (K % 64 == 0), in planes of
// 64 columns so that the 256 rows of a tile's K step are one contiguous
// 24 KiB block (with rows R apart at a large stride, the loads bound the
// K loop: at c5 the down GEMM ran 1.64 ms that way, 1.33 ms in planes):
//   codes  [K/64][srows][96] bytes: per row, block 2c then block 2c+1 of
//          plane c, each term 0 (24 bytes, element i at bits 6i..6i+5,
//          little-endian) then term 1;
//   scales [K/64][srows][4] bytes: per row and plane (block 2c term 0,
//          block 2c term 1, block 2c+1 term 0, block 2c+1 term 1);
//   srows >= R + 256 so whole-tile loads stay in bounds.
//
// Lane layout of the scaled MFMA (checked on the GPU against a host model):
// lane l supplies row l % 32, K elements 32 * (l / 32) .. + 31 of each
// operand, and byte `opsel` of its scale register scales that row's block.
// D[i][j] = sum_k src0[i][k] * src1[j][k] lands in lane j, register i as for
// the bf16 32x32 MFMAs. Weights are src0 (rows = output columns n), the
// activation terms src1 (lanes = token rows m), as in gemm.hip.
#include <algorithm>

#include "device_util.hpp"
#include "moe_internal.hpp"

namespace tmt {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x6 __attribute__((ext_vector_type(6)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

constexpr int BM = kGemmTileRows;  // 256 token rows per tile
constexpr int BN = 256;            // output columns per tile
constexpr int NST = 4;             // LDS ring stages of K = 64
// One stage: activation codes [256 rows][2 halves][48 B] (block = half ^
// bit 3 of the row), weight codes
// [256 n][2 halves][16 B] (block = half ^ bit 3 of n), activation scales
// [256 rows][4 B], weight scales [2 blocks][256 n] (a 1 KiB load; the second
// half is unused).
constexpr int A_BYTES = 2 * BM * 48;
constexpr int B_BYTES = 2 * BN * 16;
constexpr int AS_BYTES = 1024, BS_BYTES = 1024;
constexpr int STAGE = A_BYTES + B_BYTES + AS_BYTES + BS_BYTES;
constexpr int A_LOADS = A_BYTES / 1024 / 4;  // 1 KiB wave loads per wave
constexpr int B_LOADS = B_BYTES / 1024 / 4;
constexpr int DMA_PER_TILE = A_LOADS + B_LOADS + 2;  // + the wave's activation-scale rows, the weight scales
constexpr int EPR = 64, WTN = 128;  // epilogue: rows per wave and pass, wave tile width
// The bf16 epilogue stages each wave's EPR x WTN bf16 rows in ring slots 2
// and 3, so slots 0 and 1 can take the next tile's first K steps meanwhile.
constexpr int EPI_OFF = 2 * STAGE, EPI = 4 * EPR * WTN * 2;
static_assert(EPI_OFF + EPI <= NST * STAGE, "bf16 staging must fit in ring slots 2 and 3");
constexpr int LDS_BYTES = NST * STAGE;
static_assert(LDS_BYTES <= 160 * 1024, "LDS ring too large");

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// One wave-wide 16-byte-per-lane load from global memory (wave-uniform base
// plus a 32-bit per-lane byte offset) into LDS at lds_base + 16 * lane
// (lds_base wave-uniform); M0 is declared clobbered.
__device__ __forceinline__ void dma16(const void* sbase, uint32_t voff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_base) : "m0");
}
// The same with 4 bytes per lane, to LDS at lds_base + 4 * lane.
__device__ __forceinline__ void dma4(const void* sbase, uint32_t voff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_base) : "m0");
}
#pragma clang diagnostic pop
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N));
}
__device__ __forceinline__ void st16_nt(void* p, uint4 v) {
    __builtin_nontemporal_store(u32x4_t{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4_t*>(p));
}

// floor(log2(amax)) - 2, the e8m0 exponent that maps the block maximum into
// [4, 8) of e2m3's range (largest value 7.5), clamped to [-127, 127]; zero
// and subnormal maxima give -127.
__device__ __forceinline__ int mx6_exponent(float amax) {
    const int be = (int)((__float_as_uint(amax) >> 23) & 255);
    return be == 0 ? -127 : max(-127, be - 129);
}
__device__ __forceinline__ float exp2_int(int e) {  // 2^e for e in [-127, 127]
    return e >= -126 ? __uint_as_float((uint32_t)(e + 127) << 23) : __uint_as_float(0x00400000u);
}

// 32 values (natural order) to e2m3 codes at scale 2^e (six packed dwords,
// element i at bits 6i). The conversion writes its destination while it still
// reads its sources, so the sources are kept live past it: the destination
// never shares a register with them.
__device__ __forceinline__ u32x6 to_e2m3(const float* x, float scale) {
    f32x16 ev, od;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        ev[i] = x[2 * i];  // packed element 2i comes from the first operand
        od[i] = x[2 * i + 1];
    }
    u32x6 q = __builtin_amdgcn_cvt_scalef32_2xpk16_fp6_f32(ev, od, scale);
    asm volatile("" : "+v"(q) : "v"(ev), "v"(od), "v"(scale));
    return q;
}
__device__ __forceinline__ void from_e2m3(u32x6 q, float scale, float* out) {
    auto d = __builtin_amdgcn_cvt_scalef32_pk32_f32_fp6(q, scale);
    asm volatile("" : "+v"(d) : "v"(q), "v"(scale));
#pragma unroll
    for (int i = 0; i < 32; ++i) out[i] = d[i];
}

// One 32-block to two e2m3 terms: codes t0, t1 and the scale bytes.
__device__ __forceinline__ void quant_block2(const float* x, u32x6& t0, u32x6& t1, uint32_t& s0, uint32_t& s1) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
    const int e0 = mx6_exponent(amax);
    const float sc0 = exp2_int(e0);
    t0 = to_e2m3(x, sc0);
    float r[32];
    from_e2m3(t0, sc0, r);
    float amax1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        r[i] = x[i] - r[i];
        amax1 = fmaxf(amax1, fabsf(r[i]));
    }
    const int e1 = mx6_exponent(amax1);
    t1 = to_e2m3(r, exp2_int(e1));
    s0 = (uint32_t)(e0 + 127);
    s1 = (uint32_t)(e1 + 127);
}

// Store a 64-column group (two 32-blocks) of one row: 96 code bytes and the
// row's scale dword of that group.
__device__ __forceinline__ void store_group(uint8_t* codes, uint8_t* scales, const u32x6* t, const uint32_t* s) {
    uint4* dst = reinterpret_cast<uint4*>(codes);
    dst[0] = make_uint4(t[0][0], t[0][1], t[0][2], t[0][3]);
    dst[1] = make_uint4(t[0][4], t[0][5], t[1][0], t[1][1]);
    dst[2] = make_uint4(t[1][2], t[1][3], t[1][4], t[1][5]);
    dst[3] = make_uint4(t[2][0], t[2][1], t[2][2], t[2][3]);
    dst[4] = make_uint4(t[2][4], t[2][5], t[3][0], t[3][1]);
    dst[5] = make_uint4(t[3][2], t[3][3], t[3][4], t[3][5]);
    *reinterpret_cast<uint32_t*>(scales) = s[0] | (s[1] << 8) | (s[2] << 16) | (s[3] << 24);
}

// bf16 rows to MX6x2, each row rounded once and written to every slot it
// is routed to (slot_of): one thread per (row, 64-column plane), rows fastest
// so that a wave reads 64 rows of one plane and writes runs of consecutive
// slots (an expert's slots hold its tokens in token order).
__global__ __launch_bounds__(kThreads) void mx_quant_rows_kernel(MxQuantParams p) {
    const int groups = p.K / 64;
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (idx >= (int64_t)p.rows * groups) return;
    const int c = (int)(idx / p.rows), r = (int)(idx % p.rows);
    const uint4* x = reinterpret_cast<const uint4*>(p.X + (int64_t)r * p.ldx + c * 64);
    uint4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = x[i];
    float f[64];
#pragma unroll
    for (int i = 0; i < 8; ++i) unpack8(v[i], f + 8 * i);
    u32x6 t[4];
    uint32_t s[4];
    quant_block2(f, t[0], t[1], s[0], s[1]);
    quant_block2(f + 32, t[2], t[3], s[2], s[3]);
    for (int j = 0; j < p.copies; ++j) {
        const int slot = p.slot_of ? p.slot_of[(int64_t)r * p.copies + j] : r;
        store_group(p.codes + ((int64_t)c * p.srows + slot) * 96, p.scales + ((int64_t)c * p.srows + slot) * 4, t, s);
    }
}

// Weight codes to K planes: blocks of RB rows x UB units of 32 bytes (one
// unit = one row's codes of one K step; UB = min(32, K/64), RB * UB = 1024)
// through LDS, read row by row and written unit by unit, so both sides move
// runs of at least 512 bytes. Blocks of set 0 come first in the grid.
__device__ __forceinline__ void planes_shape(int K, int& ub, int& rb) {
    ub = min(32, K / 64);
    rb = 1024 / ub;
}
__global__ __launch_bounds__(kThreads) void mx_weight_planes_kernel(MxPlanesParams p, int nb0) {
    __shared__ uint4 t[2048 + 1024];  // RB rows of 2 UB uint4, one uint4 of padding per row (RB <= 1024)
    const int w = (int)blockIdx.x < nb0 ? 0 : 1;
    const int N = p.N[w], units = p.K[w] / 64;
    int ub, rb;
    planes_shape(p.K[w], ub, rb);
    const int bx = (int)blockIdx.x - (w ? nb0 : 0);
    const int ncu = (units + ub - 1) / ub, ncr = (N + rb - 1) / rb;
    const int e = bx / (ncu * ncr), rem = bx % (ncu * ncr);
    const int r0 = (rem / ncu) * rb, u0 = (rem % ncu) * ub;
    const int64_t row_bytes = p.K[w] / 2;
    const uint8_t* src = p.src[w][e];
    uint8_t* dst = p.dst[w] + (int64_t)e * N * row_bytes;
    const int nu = min(ub, units - u0), stride = 2 * ub + 1;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int q = threadIdx.x + kThreads * j, row = q / (2 * ub), hu = q % (2 * ub);
        if ((hu >> 1) < nu && r0 + row < N)
            t[row * stride + hu] = *reinterpret_cast<const uint4*>(src + (int64_t)(r0 + row) * row_bytes + u0 * 32 + hu * 16);
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int q = threadIdx.x + kThreads * j, u = q / (2 * rb), row = (q % (2 * rb)) >> 1, half = q & 1;
        if (u < nu && r0 + row < N)
            *reinterpret_cast<uint4*>(dst + ((int64_t)(u0 + u) * N + r0 + row) * 32 + half * 16) = t[row * stride + u * 2 + half];
    }
}

// QUANT_OUT: the output is SiLU(C) in MX6x2 (the next GEMM's activation);
// otherwise C in bf16. nvb virtual blocks map to tiles; a workgroup takes
// vb = blockIdx.x, blockIdx.x + gridDim.x, ... (one each when the grid holds
// all of them). With QUANT_OUT the epilogue uses no LDS, so the next tile's
// first NST K steps are requested before it and land while it runs.
template <bool QUANT_OUT>
__global__ __launch_bounds__(256, 1) void mx_gemm_kernel(MxGemmParams p, int nvb) {
    __shared__ uint4 lds_raw[LDS_BYTES / 16];
    uint8_t* lds = reinterpret_cast<uint8_t*>(lds_raw);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int ntn = (p.N + BN - 1) / BN;
    const int nk = p.K / 64;
    const int64_t a_plane = p.a_srows * 96;  // bytes per 64-column plane of the activation codes

    // ---- tiles: XCD-aware groups of 32 tiles, as in gemm.hip. Virtual block
    // vb runs on XCD vb % 8, and gridDim.x is a multiple of 8, so a workgroup
    // stays on the XCD of its groups. Blocks that hold no tile are skipped.
    const int gn = min(ntn, 8), gm = 32 / gn;
    const int ngn = (ntn + gn - 1) / gn;
    const ExpertTiles tmap = expert_tiles<BM>(p.offsets, p.E, lane);
    auto find_tile = [&](int& vb, int& nt, int& e, int& row0, int& rows) {
        for (; vb < nvb; vb += (int)gridDim.x) {
            const int lid = (((vb >> 8) << 3) + (vb & 7)) * 32 + ((vb >> 3) & 31);
            const int G = lid >> 5, gi = lid & 31;
            if (gi >= gm * gn) continue;
            const int mt = (G / ngn) * gm + gi % gm;
            nt = (G % ngn) * gn + gi / gm;
            if (nt >= ntn) continue;
            if (expert_tile<BM>(tmap, mt, e, row0, rows)) return true;
        }
        return false;
    };
    int vb = blockIdx.x, nt = 0, e = -1, row0 = 0, rows = 0;
    if (!find_tile(vb, nt, e, row0, rows)) return;

    // ---- DMA addressing: wave-uniform bases, 32-bit lane offsets ------------
    // (the host keeps every offset below 2^31). Activation codes: six
    // consecutive 16-byte slots hold one row's 96 bytes of the stage (its row
    // of the K step's plane), so the tile's 256 rows are one contiguous 24 KiB
    // block; rows row0 .. row0 + 255 are in bounds for every tile (srows >=
    // slots + 256), so these offsets do not depend on the tile. The row's two
    // 48-byte halves are swapped in LDS when bit 3 of the row is set
    // (conflict-free fragment reads).
    uint32_t a_off[A_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
        const int s = (wave * A_LOADS + i) * 64 + lane;  // 16-byte slot of the A region
        const int row = s / 6, part = s % 6;
        const int kb = (part / 3) ^ ((row >> 3) & 1), c = part % 3;
        a_off[i] = (uint32_t)(row * 96 + kb * 48 + c * 16);
    }
    // scales: wave w loads the activation scales of tile rows 64w .. 64w+63
    // (4 bytes per row and lane); every wave loads the tile's weight scales
    // (the same bytes to the same place)
    const uint32_t as_off = (uint32_t)(64 * wave + lane) * 4u;
    const uint32_t as_lds = A_BYTES + B_BYTES + 256u * (uint32_t)wave;
    constexpr uint32_t ws_lds = A_BYTES + B_BYTES + AS_BYTES;
    // Per tile: the bases, and the weight offsets. Weight codes are in K
    // planes ([K/64][N][32]), so a tile's K step is one contiguous 8 KiB
    // block: lane pair (2m, 2m+1) loads the 32 bytes (both 32-blocks) of row
    // m. In LDS the row's two 16-byte halves are swapped when bit 3 of the
    // row is set, which keeps the fragment reads (16 rows at a 32-byte stride)
    // free of bank conflicts. Rows past N are clamped to N - 1.
    const uint8_t *a_base = nullptr, *as_base = nullptr, *wq = nullptr, *wsc = nullptr;
    uint32_t b_off[B_LOADS], ws_off = 0;
    auto set_tile = [&](int t_nt, int t_e, int t_row0) {
        a_base = p.a_codes + (int64_t)t_row0 * 96;
        as_base = p.a_scales + (int64_t)t_row0 * 4;
        wq = p.wq[t_e];
        wsc = p.wsc[t_e];
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) {
            const int s = (wave * B_LOADS + i) * 64 + lane;  // 16-byte slot of the B region: row s/2, half s%2
            const int n = s >> 1, kb = (s & 1) ^ ((n >> 3) & 1);
            b_off[i] = (uint32_t)(min(t_nt * BN + n, p.N - 1) * 32 + kb * 16);
        }
        ws_off = (uint32_t)(((lane >> 4) & 1) * p.N + min(t_nt * BN + (lane & 15) * 16, p.N - 16));
    };
    const uint32_t lds0 = lds_addr(lds);
    // K step t (< nk) of the current addressing into ring slot t % NST.
    auto dma_tile = [&](int t) {
        const uint32_t sb = lds0 + (uint32_t)((t % NST) * STAGE);
        const uint8_t* ab = a_base + (int64_t)t * a_plane;
        const uint8_t* bb = wq + (int64_t)t * p.N * 32;
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) dma16(ab, a_off[i], sb + (uint32_t)(wave * A_LOADS + i) * 1024u);
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) dma16(bb, b_off[i], sb + A_BYTES + (uint32_t)(wave * B_LOADS + i) * 1024u);
        dma4(as_base + (int64_t)t * p.a_srows * 4, as_off, sb + as_lds);
        dma16(wsc + (int64_t)t * 2 * p.N, ws_off, sb + ws_lds);
    };

    // ---- fragments ----------------------------------------------------------
    // Weight codes (src0): 32 e2m1 per lane in four dwords; activation terms
    // (src1): six dwords each, read as 16 + 8 bytes (term 0) and 8 + 16
    // bytes (term 1) so that every operand lands in consecutive registers.
    const int kb = lane >> 5;
    const int b_lane = (2 * (wn * 128 + (lane & 31)) + (kb ^ ((lane >> 3) & 1))) * 16;  // + 1024 j
    const int bs_lane = A_BYTES + B_BYTES + AS_BYTES + kb * BN + wn * 128 + (lane & 31);  // + 32 j
    const int a_lane = (wm * 128 + (lane & 31)) * 96 + (kb ^ ((lane >> 3) & 1)) * 48;  // + 3072 i
    const int as_lane = A_BYTES + B_BYTES + (wm * 128 + (lane & 31)) * 4;  // + 128 i
    const int as_shift = 16 * kb;
    i32x4 bq[2][4];
    uint32_t bsc[2][4];
    i32x8 a0[4], a1[4];
    uint32_t asc[4];
    f32x16 acc[4][4];
    // B fragments of the tile in stage `sg` into register set `B`.
#define MX_LOAD_B(B, sg)                                                                              \
    do {                                                                                              \
        const uint8_t* st_ = lds + (sg) * STAGE;                                                      \
        _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                               \
            bq[B][j] = *reinterpret_cast<const i32x4*>(st_ + A_BYTES + b_lane + 1024 * j);            \
            bsc[B][j] = st_[bs_lane + 32 * j];                                                        \
        }                                                                                             \
    } while (0)
    // A fragments of row block i of the tile in stage `sg`.
#define MX_LOAD_A(i, sg)                                                                              \
    do {                                                                                              \
        const uint8_t* pa_ = lds + (sg) * STAGE + a_lane + 3072 * (i);                                \
        const i32x4 x0_ = *reinterpret_cast<const i32x4*>(pa_);                                       \
        const i32x2 x1_ = *reinterpret_cast<const i32x2*>(pa_ + 16);                                  \
        const i32x2 x2_ = *reinterpret_cast<const i32x2*>(pa_ + 24);                                  \
        const i32x4 x3_ = *reinterpret_cast<const i32x4*>(pa_ + 32);                                  \
        const i32x4 x1w_ = __builtin_shufflevector(x1_, x1_, 0, 1, -1, -1);                           \
        const i32x4 x2w_ = __builtin_shufflevector(x2_, x2_, 0, 1, -1, -1);                           \
        a0[i] = __builtin_shufflevector(x0_, x1w_, 0, 1, 2, 3, 4, 5, -1, -1);                         \
        a1[i] = __builtin_shufflevector(x2w_, x3_, 0, 1, 4, 5, 6, 7, -1, -1);                         \
        asc[i] = *reinterpret_cast<const uint32_t*>(lds + (sg) * STAGE + as_lane + 128 * (i)) >> as_shift; \
    } while (0)
    // The MFMAs of row block i with register set B.
#define MX_MMA_ROW(i, B)                                                                              \
    do {                                                                                              \
        _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                               \
            const i32x8 w_ = __builtin_shufflevector(bq[B][j], bq[B][j], 0, 1, 2, 3, -1, -1, -1, -1); \
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w_, a0[i], acc[i][j], 4, 2, 0,  \
                                                                       (int)bsc[B][j], 0, (int)asc[i]); \
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w_, a1[i], acc[i][j], 4, 2, 0,  \
                                                                       (int)bsc[B][j], 1, (int)asc[i]); \
        }                                                                                             \
    } while (0)
    // Until at most n (0..3) k64 tiles of this wave's DMA are in flight.
    auto wait_tiles = [&](int n) {
        if (n >= 3) wait_vm<3 * DMA_PER_TILE>();
        else if (n == 2) wait_vm<2 * DMA_PER_TILE>();
        else if (n == 1) wait_vm<DMA_PER_TILE>();
        else wait_vm<0>();
    };
    // One k64 tile t (stage S = t % NST, register set B = t % 2): wait for
    // tile t+1, request tile t+NST into slot S (tile t's fragments are in
    // registers since step t-1, and the barrier's LDS wait means every wave
    // has finished reading them), read tile t+1's weight fragments, and
    // refill each activation row block with tile t+1's right after its MFMAs.
    // Tiles t+2 .. t+NST stay in flight: every slot but the one being read.
#define MX_STEP(S, B)                                                                                 \
    do {                                                                                              \
        const int t_ = kt + (S);                                                                      \
        if (t_ < nk) {                                                                                \
            wait_tiles(min(NST - 2, nk - 2 - t_));                                                    \
            __syncthreads();                                                                          \
            if (t_ + NST < nk) dma_tile(t_ + NST);                                                    \
            const int sn_ = t_ + 1 < nk ? ((S) + 1) % NST : (S);                                      \
            MX_LOAD_B((B) ^ 1, sn_);                                                                  \
            MX_MMA_ROW(0, B);                                                                         \
            MX_LOAD_A(0, sn_);                                                                        \
            MX_MMA_ROW(1, B);                                                                         \
            MX_LOAD_A(1, sn_);                                                                        \
            MX_MMA_ROW(2, B);                                                                         \
            MX_LOAD_A(2, sn_);                                                                        \
            MX_MMA_ROW(3, B);                                                                         \
            MX_LOAD_A(3, sn_);                                                                        \
        }                                                                                             \
    } while (0)

    // ---- epilogue -----------------------------------------------------------
    // acc[i][j][r] = C[m][n] with m = wm*128 + 32i + (lane&31) and
    // n = wn*128 + 32j + 8(r>>2) + 4(lane>>5) + (r&3).
    const int mbase = wm * 128, nbase = wn * 128;
    // after_block(i) runs after row block i of the MX epilogue
    auto epilogue = [&](int t_row0, int t_rows, int t_nt, auto after_block) __attribute__((always_inline)) {
        const int nlim = min(BN, p.N - t_nt * BN);
        if constexpr (QUANT_OUT) {
            // SiLU and the two-term MX6 quantisation straight from the
            // accumulators: lanes l and l ^ 32 hold the two halves of each
            // 32-column block of row l % 32, and one v_permlane32_swap per register
            // pair (blocks 0 and 2, blocks 1 and 3) gives the lower half-wave all
            // of blocks 0 and 1 and the upper all of blocks 2 and 3: in both, the
            // first result of register r is element 8 (r / 4) + r % 4 of the block
            // and the second element 8 (r / 4) + 4 + r % 4. Each lane then owns
            // one (row, 64-column group) per row block, with no LDS staging.
            const int hi = lane >> 5;
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // keep the row blocks not yet converted in the accumulator
                // registers: without this the allocator copies them all into
                // VGPRs at the loop exit and spills
#pragma unroll
                for (int i2 = i; i2 < 4; ++i2)
#pragma unroll
                    for (int j = 0; j < 4; ++j) asm volatile("" : "+a"(acc[i2][j]));
                const int m = mbase + 32 * i + (lane & 31);
                const int n = nbase + 64 * hi;
                const bool in = m < t_rows && n < nlim;
                const int slot = t_row0 + m;
                const int col = t_nt * BN + n;  // multiple of 64
                uint4* codes = reinterpret_cast<uint4*>(p.q_codes + ((int64_t)(col / 64) * p.q_srows + slot) * 96);
                uint32_t sc = 0;
#pragma unroll
                for (int b = 0; b < 2; ++b) {  // one 32-column block at a time
                    float x[32];
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int e = 8 * (r >> 2) + (r & 3);
                        const u32x2_t sw = __builtin_amdgcn_permlane32_swap(
                            __float_as_uint(acc[i][b][r]), __float_as_uint(acc[i][b + 2][r]), false, false);
                        x[e] = silu_fast(__uint_as_float(sw[0]));
                        x[e + 4] = silu_fast(__uint_as_float(sw[1]));
                    }
                    u32x6 t0, t1;
                    uint32_t s0, s1;
                    quant_block2(x, t0, t1, s0, s1);
                    sc |= (s0 | (s1 << 8)) << (16 * b);
                    if (in) {  // the block's 48 code bytes: t0 then t1
                        codes[3 * b + 0] = make_uint4(t0[0], t0[1], t0[2], t0[3]);
                        codes[3 * b + 1] = make_uint4(t0[4], t0[5], t1[0], t1[1]);
                        codes[3 * b + 2] = make_uint4(t1[2], t1[3], t1[4], t1[5]);
                    }
                }
                if (in) *reinterpret_cast<uint32_t*>(p.q_scales + ((int64_t)(col / 64) * p.q_srows + slot) * 4) = sc;
                after_block(i);
                __builtin_amdgcn_sched_barrier(0);  // one row block's values live at a time
            }
        } else {
            // bf16 C: rounded once and staged per wave as bf16 rows [EPR][WTN]
            // (16-byte chunks swizzled by row) in ring slots 2 and 3, two
            // passes; every row leaves as 16 lanes x 16 bytes.
            constexpr int CH = WTN / 8;  // 16-byte chunks per staged row
            uint8_t* stage_b = lds + EPI_OFF + wave * (EPR * WTN * 2);
#pragma unroll
            for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
                for (int ii = 0; ii < 2; ++ii) {
                    const int i = pass * 2 + ii;
                    const int lr = ii * 32 + (lane & 31);
                    // the row blocks not yet staged stay in the accumulator registers
#pragma unroll
                    for (int i2 = i; i2 < 4; ++i2)
#pragma unroll
                        for (int j = 0; j < 4; ++j) asm volatile("" : "+a"(acc[i2][j]));
#pragma unroll
                    for (int j = 0; j < 4; ++j)
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            // columns 32j + 8q + 4(lane / 32) .. + 3: half (lane / 32) of chunk 4j + q
                            const int ch = j * 4 + q;
                            *reinterpret_cast<uint2*>(stage_b + lr * (WTN * 2) + ((ch ^ (lr & (CH - 1))) * 16) + (lane >> 5) * 8) =
                                make_uint2(pack_bf2(acc[i][j][4 * q], acc[i][j][4 * q + 1]),
                                           pack_bf2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]));
                        }
                }
                __syncthreads();
                {
                    constexpr int LPR = WTN / 8, RPI = 64 / LPR;  // lanes per row, rows per instruction
                    uint16_t* C = p.c;
                    const int cl = lane % LPR;
                    const int n = nbase + cl * 8;
#pragma unroll
                    for (int k = 0; k < EPR / RPI; ++k) {
                        const int rr = lane / LPR + RPI * k;
                        const int m = mbase + pass * EPR + rr;
                        if (m >= t_rows || n >= nlim) continue;
                        const uint4 v = *reinterpret_cast<const uint4*>(stage_b + rr * (WTN * 2) + ((cl ^ (rr & (CH - 1))) * 16));
                        st16_nt(C + (int64_t)(t_row0 + m) * p.ldc + t_nt * BN + n, v);
                    }
                }
                __syncthreads();
            }
        }
    };

    set_tile(nt, e, row0);
    bool prefetched = false;
    int late = 0;
    for (;;) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
        // ---- main loop, unrolled by the ring depth so that every stage index
        // is a compile-time constant ------------------------------------------
        if (!prefetched) {
#pragma unroll
            for (int t = 0; t < NST; ++t)
                if (t < nk) dma_tile(t);
            wait_tiles(min(NST, nk) - 1);
        } else {
            // the K steps requested before the last epilogue's stores (and
            // those stores); `late` K steps went out after them
            wait_tiles(late);
        }
        __syncthreads();
        MX_LOAD_B(0, 0);
        MX_LOAD_A(0, 0);
        MX_LOAD_A(1, 0);
        MX_LOAD_A(2, 0);
        MX_LOAD_A(3, 0);
        for (int kt = 0; kt < nk; kt += NST) {
            MX_STEP(0, 0);
            MX_STEP(1, 1);
            MX_STEP(2, 0);
            MX_STEP(3, 1);
        }
        __syncthreads();  // every wave has read its last fragments: the ring is free

        // the workgroup's next tile: its first NST K steps load around the
        // epilogue. Two go out before it; with QUANT_OUT one after each of its
        // first two row blocks (a burst of all four slowed the epilogue's own
        // stores), in bf16 after it (it stages through slots 2 and 3).
        int vb2 = vb + (int)gridDim.x, nt2 = 0, e2 = -1, row02 = 0, rows2 = 0;
        const bool more = find_tile(vb2, nt2, e2, row02, rows2);
        if (more) {
            set_tile(nt2, e2, row02);
            dma_tile(0);
            if (1 < nk) dma_tile(1);
        }
        epilogue(row0, rows, nt, [&](int i) {
            if (QUANT_OUT && more && i < 2 && i + 2 < nk) dma_tile(i + 2);
        });
        late = 0;
        if (!QUANT_OUT && more) {
#pragma unroll
            for (int t = 2; t < NST; ++t)
                if (t < nk) {
                    dma_tile(t);
                    ++late;
                }
        }
        if (!more) break;
        vb = vb2;
        nt = nt2;
        e = e2;
        row0 = row02;
        rows = rows2;
        prefetched = true;
    }
#undef MX_STEP
#undef MX_MMA_ROW
#undef MX_LOAD_A
#undef MX_LOAD_B
}

}  // namespace

hipError_t launch_mx_weight_planes(const MxPlanesParams& p, hipStream_t s) {
    if (p.E <= 0) return hipSuccess;
    if (p.E > kMaxExperts) return hipErrorInvalidValue;
    int64_t nb[2] = {0, 0};
    for (int w = 0; w < 2; ++w) {
        if (p.N[w] == 0) continue;  // an empty set
        if (p.N[w] < 0 || p.N[w] % 32 != 0 || p.K[w] <= 0 || p.K[w] % 64 != 0) return hipErrorInvalidValue;
        const int ub = std::min(32, p.K[w] / 64), rb = 1024 / ub;
        nb[w] = (int64_t)p.E * ((p.K[w] / 64 + ub - 1) / ub) * ((p.N[w] + rb - 1) / rb);
    }
    if (nb[0] + nb[1] > 0x7fffffff) return hipErrorInvalidValue;
    if (nb[0] + nb[1] == 0) return hipSuccess;
    mx_weight_planes_kernel<<<(unsigned)(nb[0] + nb[1]), kThreads, 0, s>>>(p, (int)nb[0]);
    return hipGetLastError();
}

hipError_t launch_mx_quant_rows(const MxQuantParams& p, hipStream_t s) {
    if (p.rows <= 0) return hipSuccess;
    if (p.K % 64 != 0 || p.copies < 1 || (!p.slot_of && p.copies != 1) || p.srows < (int64_t)p.rows * p.copies)
        return hipErrorInvalidValue;
    const int64_t items = (int64_t)p.rows * (p.K / 64);
    mx_quant_rows_kernel<<<(unsigned)((items + kThreads - 1) / kThreads), kThreads, 0, s>>>(p);
    return hipGetLastError();
}

hipError_t launch_mx_gemm(bool quant_out, const MxGemmParams& p, hipStream_t s) {
    if (p.slots <= 0) return hipSuccess;
    if (p.K % 64 != 0 || p.K <= 0 || p.N % 64 != 0 || p.N <= 0) return hipErrorInvalidValue;
    // lane offsets into one activation plane and into the weights are 32-bit
    if (p.a_srows * 96 > 0x7fffffffLL || (int64_t)p.N * (p.K / 2) > 0x7fffffffLL) return hipErrorInvalidValue;
    const int64_t ntn = (p.N + BN - 1) / BN;
    const int64_t gn = ntn < 8 ? ntn : 8, gm = 32 / gn;
    const int64_t ngn = (ntn + gn - 1) / gn;
    const int64_t mtiles = (int64_t)(p.slots + BM - 1) / BM + p.E;  // >= sum_e ceil(cnt_e / BM)
    const int64_t groups = ((mtiles + gm - 1) / gm) * ngn;
    const int64_t grid = (groups * 32 + 255) / 256 * 256;
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    // persistent: one workgroup per CU (a multiple of 8, so each keeps its XCD)
    const int64_t cus = cu_count() / 8 * 8;
    const int64_t g = cus >= 8 && cus < grid ? cus : grid;
    if (quant_out) mx_gemm_kernel<true><<<(unsigned)g, 256, 0, s>>>(p, (int)grid);
    else mx_gemm_kernel<false><<<(unsigned)g, 256, 0, s>>>(p, (int)grid);
    return hipGetLastError();
}

}  // namespace tmt
