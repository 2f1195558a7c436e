// gemm.hip -- grouped bf16 MFMA GEMMs over expert segments (gfx950).
//
// Replaces the reference's per-expert cuBLAS loops (tmt-cuda/src/moe.cu:431-436
// forward, :533-539 backward; wrappers tmt-cuda/src/linalg.cu:9-41) and the
// gather kernel (moe.cu:127-140): one launch covers all experts, tiles are
// found from the device-side offset table (no host sync, no 128-row padding),
// and the token gather is folded into the operand loads.
//
// Tile: 256 x 256 outputs per 256-thread workgroup (one workgroup per CU),
// 4 waves in 2 x 2, each wave 128 x 128 = 4 x 4 v_mfma_f32_32x32x16_bf16
// tiles (256 fp32 accumulators per lane). K step 64 with two 64 KiB LDS
// stages. Per K step a wave reads 32 KiB of fragments for 2 MFLOP, half the
// LDS traffic per flop of a 64 x 64 wave tile.
//
// Operands are staged in LDS as [rows][64] bf16, K contiguous, 16-byte chunks
// XOR-swizzled by (row ^ row>>3) & 7: fragment reads and both kinds of stores
// are bank-conflict free. Operands whose memory layout has the row index
// contiguous (weights read as [K][N] in backward, token-major activations in
// the weight-gradient GEMMs) are transposed in registers: a thread loads an
// 8 x 8 block with eight 16-byte loads and stores eight K-contiguous rows.
// Global loads for step k+2 are in flight while step k computes.
//
// Epilogue: accumulators go through LDS (fp32, 16-byte chunks swizzled by
// row) so every global store is a 16-byte vector and each output row is
// written as one contiguous 256-byte (bf16) or 512-byte (fp32) run.
#include "device_util.hpp"
#include "moe_internal.hpp"

namespace tmt {
namespace {

constexpr int BK = 64;
constexpr int BM = 256;
constexpr int BN = 256;
constexpr int WTM = 128, WTN = 128;       // wave tile
constexpr int MI = WTM / 32, NJ = WTN / 32;
constexpr int STAGE = (BM + BN) * BK;     // bf16 elements per LDS stage

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int KIND> struct Traits;
// C[slot][n] = X[perm[slot]] . W_up[e][n]         A: K-contig gather, B: K-contig
template <> struct Traits<GEMM_UP> {
    static constexpr bool group_k = false, a_kc = true, b_kc = true, gather = true;
};
// C[slot][n] = A[slot] . W_down[e][n]
template <> struct Traits<GEMM_DOWN> {
    static constexpr bool group_k = false, a_kc = true, b_kc = true, gather = false;
};
// C[slot][n] = (dO[slot] . W_down[e][:, n]) * silu'(U)   B is [K][N]
template <> struct Traits<GEMM_DACT> {
    static constexpr bool group_k = false, a_kc = true, b_kc = false, gather = false;
};
// C[slot][n] = dU[slot] . W_up[e][:, n]            B is [K][N]
template <> struct Traits<GEMM_DX> {
    static constexpr bool group_k = false, a_kc = true, b_kc = false, gather = false;
};
// dW_down[e][m][n] = sum_slot dO[slot][m] * A[slot][n]
template <> struct Traits<GEMM_DW_DOWN> {
    static constexpr bool group_k = true, a_kc = false, b_kc = false, gather = false;
};
// dW_up[e][m][n] = sum_slot dU[slot][m] * X[perm[slot]][n]
template <> struct Traits<GEMM_DW_UP> {
    static constexpr bool group_k = true, a_kc = false, b_kc = false, gather = true;
};

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row ^ (row >> 3)) & 7); }

__device__ __forceinline__ uint32_t comp(const uint4& v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// Element i (0..7) of eight 8-element rows st[0..7] -> one 8-element column.
__device__ __forceinline__ uint4 column8(const uint4* st, int i) {
    uint32_t d[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t a = comp(st[2 * q], i >> 1), b = comp(st[2 * q + 1], i >> 1);
        d[q] = (i & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
    }
    return make_uint4(d[0], d[1], d[2], d[3]);
}

__device__ __forceinline__ uint4 ld16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }

template <int KIND, bool DUAL>
__global__ __launch_bounds__(kThreads, 1) void grouped_gemm_kernel(GemmParams p) {
    using Tr = Traits<KIND>;
    __shared__ uint4 lds_raw[2 * STAGE / 8];
    uint16_t* lds = reinterpret_cast<uint16_t*>(lds_raw);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int ntn = (p.N + BN - 1) / BN;

    // ---- tile coordinates -------------------------------------------------
    // The hardware hands workgroup b to XCD b % 8 and each XCD runs 32 at a
    // time (one per CU). Workgroups b = 8j + x with j in [32t, 32t + 32) are
    // therefore co-resident on XCD x; they get the 32 tiles of group
    // G = 8t + x, laid out as gm x gn tiles (gn = min(tiles across N, 8)) so
    // that the XCD's L2 serves each operand slice to several workgroups.
    // Consecutive groups go to different XCDs, which spreads the long tiles
    // of the weight-gradient GEMMs (experts in descending-count order).
    const int lid = ((((int)blockIdx.x >> 8) << 3) + ((int)blockIdx.x & 7)) * 32 + (((int)blockIdx.x >> 3) & 31);
    const int G = lid >> 5, gi = lid & 31;
    const int gn = min(ntn, 8), gm = 32 / gn;
    const int ngn = (ntn + gn - 1) / gn;
    if (gi >= gm * gn) return;
    int e = -1, mt = 0, nt = 0;
    int row0 = 0, rows = 0;   // activation GEMMs: slot range of this tile
    int kbeg = 0, kend = 0;   // reduction range (slots for dW GEMMs)
    int mlim = 0;             // valid output rows in this tile
    if constexpr (!Tr::group_k) {
        mt = (G / ngn) * gm + gi % gm;
        nt = (G % ngn) * gn + gi / gm;
        if (nt >= ntn) return;
        int t0 = 0;
        for (int ee = 0; ee < p.E; ++ee) {
            const int beg = p.offsets[ee], end = p.offsets[ee + 1];
            const int tiles = (end - beg + BM - 1) / BM;
            if (mt < t0 + tiles) {
                e = ee;
                row0 = beg + (mt - t0) * BM;
                rows = min(BM, end - row0);
                break;
            }
            t0 += tiles;
        }
        if (e < 0) return;  // beyond the last tile of the last expert
        kbeg = 0;
        kend = p.K;
        mlim = rows;
    } else {
        const int ntm = (p.M + BM - 1) / BM;
        const int gpe = ((ntm + gm - 1) / gm) * ngn;  // groups per expert
        const int ei = G / gpe, g = G - ei * gpe;
        if (ei >= p.E) return;
        mt = (g / ngn) * gm + gi % gm;
        nt = (g % ngn) * gn + gi / gm;
        if (mt >= ntm || nt >= ntn) return;
        e = p.order[ei];
        kbeg = p.offsets[e];
        kend = p.offsets[e + 1];
        mlim = min(BM, p.M - mt * BM);
    }
    const int nlim = min(BN, p.N - nt * BN);  // valid output columns in this tile
    const int nk = (kend - kbeg + BK - 1) / BK;

    // ---- loaders: every thread stages 8 vectors of each operand ------------
    // K-contiguous: rows kc_r + 32i, 16-byte chunk kc_ch.
    // Row-contiguous: columns 8*mc_c8 .. +7, k rows 8*mc_kg .. +7.
    const int kc_ch = tid & 7, kc_r = tid >> 3;
    const int mc_c8 = tid & 31, mc_kg = tid >> 5;

    // Row/column indices past the valid range are clamped to a valid address
    // instead of masked: they only feed output rows or columns that the
    // epilogue does not store. Only the reduction tail of the weight-gradient
    // GEMMs (slots past the expert segment) must read as zero; it is masked
    // with an all-ones/zero word that the compiler cannot turn into a branch.
    const uint16_t* a_rp[8];
    const uint16_t* b_rp[8];
    const uint16_t* a_mc = nullptr;
    const uint16_t* b_mc = nullptr;
    int b_src[8];  // gathered source rows of the next B tile (dW_up)

    if constexpr (Tr::a_kc) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int slot = min(row0 + kc_r + 32 * i, p.slots - 1);
            const int src = Tr::gather ? p.perm[slot] : slot;
            a_rp[i] = p.a + (int64_t)src * p.lda + kc_ch * 8;
        }
    } else {
        a_mc = p.a + min(mt * BM + mc_c8 * 8, p.M - 8);
    }
    if constexpr (Tr::b_kc) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int n = min(nt * BN + kc_r + 32 * i, p.N - 1);
            b_rp[i] = p.w[e] + (int64_t)n * p.ldb + kc_ch * 8;
        }
    } else if constexpr (!Tr::group_k) {
        b_mc = p.w[e] + min(nt * BN + mc_c8 * 8, p.N - 8);  // weight read as [K][N]
    } else {
        b_mc = p.b + min(nt * BN + mc_c8 * 8, p.N - 8);
    }

    auto fetch_src = [&](int k0) {
        if constexpr (Tr::group_k && Tr::gather) {
#pragma unroll
            for (int t = 0; t < 8; ++t) b_src[t] = p.perm[min(k0 + mc_kg * 8 + t, kend - 1)];
        }
    };
    auto tail_mask = [&](int k) {
        uint32_t m = k < kend ? 0xffffffffu : 0u;
        asm("" : "+v"(m));
        return m;
    };
    auto and4 = [](uint4 v, uint32_t m) { return make_uint4(v.x & m, v.y & m, v.z & m, v.w & m); };

    uint4 sa[8], sb[8];
    auto gload = [&](int k0) {
        if constexpr (Tr::a_kc) {
#pragma unroll
            for (int i = 0; i < 8; ++i) sa[i] = ld16(a_rp[i] + k0);
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int k = k0 + mc_kg * 8 + t;
                sa[t] = and4(ld16(a_mc + (int64_t)min(k, kend - 1) * p.lda), tail_mask(k));
            }
        }
        if constexpr (Tr::b_kc) {
#pragma unroll
            for (int i = 0; i < 8; ++i) sb[i] = ld16(b_rp[i] + k0);
        } else if constexpr (Tr::group_k && Tr::gather) {
#pragma unroll
            for (int t = 0; t < 8; ++t)
                sb[t] = and4(ld16(b_mc + (int64_t)b_src[t] * p.ldb), tail_mask(k0 + mc_kg * 8 + t));
            fetch_src(k0 + BK);  // source rows of the next tile, off the critical path
        } else if constexpr (Tr::group_k) {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int k = k0 + mc_kg * 8 + t;
                sb[t] = and4(ld16(b_mc + (int64_t)min(k, kend - 1) * p.ldb), tail_mask(k));
            }
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) sb[t] = ld16(b_mc + (int64_t)(k0 + mc_kg * 8 + t) * p.ldb);
        }
    };
    // Store half `hf` (vectors 4hf..4hf+3) of the staged tile into LDS stage.
    auto lstore_half = [&](int stage, int hf) {
        uint16_t* ta = lds + stage * STAGE;
        uint16_t* tb = ta + BM * BK;
#pragma unroll
        for (int i = 4 * hf; i < 4 * hf + 4; ++i) {
            if constexpr (Tr::a_kc) {
                const int r = kc_r + 32 * i;
                *reinterpret_cast<uint4*>(ta + r * BK + swz(r, kc_ch) * 8) = sa[i];
            } else {
                const int r = mc_c8 * 8 + i;
                *reinterpret_cast<uint4*>(ta + r * BK + swz(r, mc_kg) * 8) = column8(sa, i);
            }
            if constexpr (Tr::b_kc) {
                const int r = kc_r + 32 * i;
                *reinterpret_cast<uint4*>(tb + r * BK + swz(r, kc_ch) * 8) = sb[i];
            } else {
                const int r = mc_c8 * 8 + i;
                *reinterpret_cast<uint4*>(tb + r * BK + swz(r, mc_kg) * 8) = column8(sb, i);
            }
        }
    };

    f32x16 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // Fragments of one k16 step: A rows wm*128 + 32i + lane%32, B rows
    // wn*128 + 32j + lane%32, 16-byte chunk 2s + lane/32.
    struct Frag {
        uint4 a[MI], b[NJ];
    };
    auto load_frag = [&](Frag& f, const uint16_t* tA, int s) {
        const uint16_t* tB = tA + BM * BK;
        const int chunk = s * 2 + (lane >> 5);
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const int r = wm * WTM + i * 32 + (lane & 31);
            f.a[i] = *reinterpret_cast<const uint4*>(tA + r * BK + swz(r, chunk) * 8);
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int r = wn * WTN + j * 32 + (lane & 31);
            f.b[j] = *reinterpret_cast<const uint4*>(tB + r * BK + swz(r, chunk) * 8);
        }
    };
    auto mma = [&](const Frag& f) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    __builtin_bit_cast(bf16x8, f.b[j]), __builtin_bit_cast(bf16x8, f.a[i]),
                    acc[i][j], 0, 0, 0);
    };

    if (nk > 0) {
        fetch_src(kbeg);
        gload(kbeg);
        lstore_half(0, 0);
        lstore_half(0, 1);
        const int last_k0 = kbeg + (nk - 1) * BK;  // prefetches past the end re-read it
        gload(min(kbeg + BK, last_k0));
        __syncthreads();
        Frag f0, f1;
        for (int kt = 0; kt < nk; ++kt) {
            const uint16_t* tA = lds + (kt & 1) * STAGE;
            const int nxt = (kt + 1) & 1;
            // The loop body is one basic block; the scheduling groups below pin
            // the order: fragments for step s+1 are read while step s's 16
            // MFMAs run, the next tile's LDS stores and the global loads of the
            // tile after it are interleaved one per MFMA. Stores into the idle
            // stage after the last tile are harmless.
            load_frag(f0, tA, 0);
            load_frag(f1, tA, 1);
            __builtin_amdgcn_sched_barrier(0);
            mma(f0);
            lstore_half(nxt, 0);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
            __builtin_amdgcn_sched_barrier(0);
            load_frag(f0, tA, 2);
            mma(f1);
            lstore_half(nxt, 1);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);  // DS read
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);  // MFMA
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x200, 1, 1);  // DS write
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);  // MFMA
            }
            __builtin_amdgcn_sched_barrier(0);
            load_frag(f1, tA, 3);
            mma(f0);
            gload(min(kbeg + (kt + 2) * BK, last_k0));
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 2);  // DS read
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 2);  // MFMA
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x020, 2, 2);  // VMEM read
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 2);  // MFMA
            }
            __builtin_amdgcn_sched_barrier(0);
            mma(f1);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
        }
    }

    // ---- epilogue ---------------------------------------------------------
    // acc[i][j][r] = C[m][n] with m = wm*128 + 32i + (lane&31) and
    // n = wn*128 + 32j + 8(r>>2) + 4(lane>>5) + (r&3). Two passes of 64 rows per
    // wave go through a 32 KiB fp32 LDS region ([64][128], 16-byte chunks
    // swizzled by row & 31), then leave as row-contiguous 16-byte stores.
    float* stage_f = reinterpret_cast<float*>(lds_raw) + wave * (64 * 128);
    const int mbase = wm * WTM, nbase = wn * WTN;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
            const int i = pass * 2 + ii;
            const int lr = ii * 32 + (lane & 31);
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int ch = j * 8 + 2 * q + (lane >> 5);
                    *reinterpret_cast<f32x4*>(stage_f + lr * 128 + ((ch ^ (lr & 31)) * 4)) =
                        f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                              acc[i][j][4 * q + 3]};
                }
        }
        __syncthreads();
        if constexpr (!Tr::group_k) {
            // 16 lanes per row (8 bf16 each), 4 rows per instruction
            uint16_t* C = reinterpret_cast<uint16_t*>(p.c);
            const int cl = lane & 15;
#pragma unroll 4
            for (int rr = lane >> 4; rr < 64; rr += 4) {
                const int m = mbase + pass * 64 + rr;
                const int n = nbase + cl * 8;
                if (m >= mlim || n >= nlim) continue;
                const float* src = stage_f + rr * 128;
                const f32x4 v0 = *reinterpret_cast<const f32x4*>(src + (((2 * cl) ^ (rr & 31)) * 4));
                const f32x4 v1 = *reinterpret_cast<const f32x4*>(src + (((2 * cl + 1) ^ (rr & 31)) * 4));
                float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                const int64_t off = (int64_t)(row0 + m) * p.ldc + nt * BN + n;
                if constexpr (KIND == GEMM_DACT) {
                    float u[8];
                    unpack8(ld16(p.u + off), u);
#pragma unroll
                    for (int t = 0; t < 8; ++t) v[t] *= dsilu_fast(u[t]);
                }
                *reinterpret_cast<uint4*>(C + off) = pack8(v);
                if constexpr (DUAL) {
#pragma unroll
                    for (int t = 0; t < 8; ++t) v[t] = silu_fast(v[t]);
                    *reinterpret_cast<uint4*>(p.c2 + off) = pack8(v);
                }
            }
        } else {
            // 32 lanes per row (4 fp32 each), 2 rows per instruction
            float* C = p.dw[e];
            const int cl = lane & 31;
#pragma unroll 4
            for (int rr = lane >> 5; rr < 64; rr += 2) {
                const int m = mbase + pass * 64 + rr;
                const int n = nbase + cl * 4;
                if (m >= mlim || n >= nlim) continue;
                const f32x4 v = *reinterpret_cast<const f32x4*>(stage_f + rr * 128 + ((cl ^ (rr & 31)) * 4));
                *reinterpret_cast<f32x4*>(C + (int64_t)(mt * BM + m) * p.ldc + nt * BN + n) = v;
            }
        }
        __syncthreads();
    }
}

}  // namespace

hipError_t launch_gemm(GemmKind kind, bool dual, const GemmParams& p, hipStream_t s) {
    if (p.N % 8 != 0 || p.N <= 0) return hipErrorInvalidValue;
    dim3 block(kThreads);
    const bool group_k = kind == GEMM_DW_DOWN || kind == GEMM_DW_UP;
    const int64_t ntn = (p.N + BN - 1) / BN;
    const int64_t gn = ntn < 8 ? ntn : 8, gm = 32 / gn;
    const int64_t ngn = (ntn + gn - 1) / gn;
    int64_t groups;
    if (group_k) {
        if (p.M % 8 != 0 || p.M <= 0) return hipErrorInvalidValue;
        const int64_t ntm = (p.M + BM - 1) / BM;
        groups = (int64_t)p.E * ((ntm + gm - 1) / gm) * ngn;
    } else {
        if (p.K % BK != 0) return hipErrorInvalidValue;
        // sum_e ceil(cnt_e / BM) <= ceil(slots / BM) + E - 1
        const int64_t mtiles = (int64_t)(p.slots + BM - 1) / BM + p.E;
        groups = ((mtiles + gm - 1) / gm) * ngn;
    }
    // whole rounds of 8 XCDs x 32 workgroups keep the block -> tile map a bijection
    const int64_t grid = (groups * 32 + 255) / 256 * 256;
    if (grid <= 0) return hipSuccess;
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    const unsigned g = (unsigned)grid;
    switch (kind) {
        case GEMM_UP:
            if (dual) grouped_gemm_kernel<GEMM_UP, true><<<g, block, 0, s>>>(p);
            else grouped_gemm_kernel<GEMM_UP, false><<<g, block, 0, s>>>(p);
            break;
        case GEMM_DOWN: grouped_gemm_kernel<GEMM_DOWN, false><<<g, block, 0, s>>>(p); break;
        case GEMM_DACT: grouped_gemm_kernel<GEMM_DACT, false><<<g, block, 0, s>>>(p); break;
        case GEMM_DX: grouped_gemm_kernel<GEMM_DX, false><<<g, block, 0, s>>>(p); break;
        case GEMM_DW_DOWN: grouped_gemm_kernel<GEMM_DW_DOWN, false><<<g, block, 0, s>>>(p); break;
        case GEMM_DW_UP: grouped_gemm_kernel<GEMM_DW_UP, false><<<g, block, 0, s>>>(p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace tmt
