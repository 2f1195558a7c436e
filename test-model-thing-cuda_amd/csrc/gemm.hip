// gemm.hip -- grouped bf16 MFMA GEMMs over expert segments (gfx950).
//
// Replaces the reference's per-expert cuBLAS loops (tmt-cuda/src/moe.cu:431-436
// forward, :533-539 backward; wrappers tmt-cuda/src/linalg.cu:9-41) and the
// gather kernel (moe.cu:127-140): one launch covers all experts, tiles are
// found from the device-side offset table (no host sync, no 128-row padding),
// and the token gather is folded into the operand loads.
//
// Tile: 128 x 128 outputs per 256-thread workgroup, 4 waves in 2 x 2, each
// wave 64 x 64 with v_mfma_f32_16x16x32_bf16; K step 64, two LDS stages.
// Both operands are staged in LDS as [rows][64] bf16 with K contiguous, 16-byte
// chunks XOR-swizzled by (row ^ row>>3) & 7 so that MFMA fragment reads and
// both kinds of stores are free of bank conflicts. Operands whose memory
// layout has the row index contiguous (weights read as [K][N] in backward,
// token-major activations in the weight-gradient GEMMs) are transposed in
// registers: each thread loads an 8x8 block with eight 16-byte loads and
// writes eight K-contiguous 16-byte rows.
//
// The MFMA takes the N-side fragment as its first operand, so each lane ends
// with 4 consecutive output columns of one row (8- or 16-byte stores).
#include "device_util.hpp"
#include "moe_internal.hpp"

namespace tmt {
namespace {

constexpr int BK = 64;
constexpr int BM = 128;
constexpr int BN = 128;

enum Epi { EPI_BF16 = 0, EPI_SILU_DUAL = 1, EPI_DSILU = 2, EPI_F32 = 3 };

template <int KIND> struct Traits;
// C[slot][n] = X[perm[slot]] . W_up[e][n]         A: K-contig gather, B: K-contig
template <> struct Traits<GEMM_UP> {
    static constexpr bool group_k = false, a_kc = true, b_kc = true, a_gather = true, b_gather = false;
};
// C[slot][n] = A[slot] . W_down[e][n]
template <> struct Traits<GEMM_DOWN> {
    static constexpr bool group_k = false, a_kc = true, b_kc = true, a_gather = false, b_gather = false;
};
// C[slot][n] = (dO[slot] . W_down[e][:, n]) * silu'(U)   B is [K][N]
template <> struct Traits<GEMM_DACT> {
    static constexpr bool group_k = false, a_kc = true, b_kc = false, a_gather = false, b_gather = false;
};
// C[slot][n] = dU[slot] . W_up[e][:, n]            B is [K][N]
template <> struct Traits<GEMM_DX> {
    static constexpr bool group_k = false, a_kc = true, b_kc = false, a_gather = false, b_gather = false;
};
// dW_down[e][m][n] = sum_slot dO[slot][m] * A[slot][n]
template <> struct Traits<GEMM_DW_DOWN> {
    static constexpr bool group_k = true, a_kc = false, b_kc = false, a_gather = false, b_gather = false;
};
// dW_up[e][m][n] = sum_slot dU[slot][m] * X[perm[slot]][n]
template <> struct Traits<GEMM_DW_UP> {
    static constexpr bool group_k = true, a_kc = false, b_kc = false, a_gather = false, b_gather = true;
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

template <int KIND, bool DUAL>
__global__ __launch_bounds__(kThreads, 2) void grouped_gemm_kernel(GemmParams p) {
    using Tr = Traits<KIND>;
    constexpr int WTM = BM / 2, WTN = BN / 2;
    constexpr int MI = WTM / 16, NJ = WTN / 16;
    constexpr int STAGE = (BM + BN) * BK;  // bf16 elements per LDS stage
    __shared__ uint4 lds_raw[2 * STAGE / 8];
    uint16_t* lds = reinterpret_cast<uint16_t*>(lds_raw);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int ntn = p.N / BN;

    // ---- tile coordinates -------------------------------------------------
    int e = -1, mt = 0, nt = 0;
    int row0 = 0, rows = 0;   // activation GEMMs: slot range of this tile
    int kbeg = 0, kend = 0;   // reduction range (slots for dW GEMMs)
    if constexpr (!Tr::group_k) {
        const int bid = blockIdx.x;
        mt = bid / ntn;
        nt = bid - mt * ntn;
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
    } else {
        const int ntm = p.M / BM;
        const int per = ntm * ntn;
        const int ei = blockIdx.x / per;
        const int rem = blockIdx.x - ei * per;
        mt = rem / ntn;
        nt = rem - mt * ntn;
        e = p.order[ei];
        kbeg = p.offsets[e];
        kend = p.offsets[e + 1];
    }
    const int nk = (kend - kbeg + BK - 1) / BK;

    // ---- loader roles: waves 0-1 stage operand A (M side), 2-3 operand B --
    const bool is_a = tid < 128;
    const int lt = tid & 127;
    const bool kc = is_a ? Tr::a_kc : Tr::b_kc;
    // K-contiguous loader: 8 rows (lt/8 + 16i), 16-byte chunk lt%8.
    const int kc_ch = lt & 7, kc_r = lt >> 3;
    const uint16_t* rp[8];
    // Row-contiguous loader: columns 8*(lt%16).., k rows 8*(lt/16)..
    const int mc_c8 = lt & 15, mc_kg = lt >> 4;
    const uint16_t* mc_base = nullptr;
    int64_t mc_ld = 0;
    const int32_t* mc_gather = nullptr;

    if (is_a) {
        if constexpr (Tr::a_kc) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int r = kc_r + 16 * i;
                rp[i] = nullptr;
                if (r < rows) {
                    const int slot = row0 + r;
                    const int src = Tr::a_gather ? p.perm[slot] : slot;
                    rp[i] = p.a + (int64_t)src * p.lda + kc_ch * 8;
                }
            }
        } else {
            mc_base = p.a + mt * BM + mc_c8 * 8;
            mc_ld = p.lda;
        }
    } else {
        if constexpr (Tr::b_kc) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                rp[i] = p.w[e] + (int64_t)(nt * BN + kc_r + 16 * i) * p.ldb + kc_ch * 8;
        } else if constexpr (!Tr::group_k) {
            mc_base = p.w[e] + nt * BN + mc_c8 * 8;  // weight read as [K][N]
            mc_ld = p.ldb;
        } else {
            mc_base = p.b + nt * BN + mc_c8 * 8;
            mc_ld = p.ldb;
            if (Tr::b_gather) mc_gather = p.perm;
        }
    }

    uint4 st[8];
    auto gload = [&](int k0) {
        if (kc) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                st[i] = rp[i] ? *reinterpret_cast<const uint4*>(rp[i] + k0) : make_uint4(0, 0, 0, 0);
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int k = k0 + mc_kg * 8 + t;
                uint4 v = make_uint4(0, 0, 0, 0);
                if (k < kend) {
                    const int src = mc_gather ? mc_gather[k] : k;
                    v = *reinterpret_cast<const uint4*>(mc_base + (int64_t)src * mc_ld);
                }
                st[t] = v;
            }
        }
    };
    auto lstore = [&](int stage) {
        uint16_t* tile = lds + stage * STAGE + (is_a ? 0 : BM * BK);
        if (kc) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int r = kc_r + 16 * i;
                *reinterpret_cast<uint4*>(tile + r * BK + swz(r, kc_ch) * 8) = st[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int r = mc_c8 * 8 + i;
                *reinterpret_cast<uint4*>(tile + r * BK + swz(r, mc_kg) * 8) = column8(st, i);
            }
        }
    };

    f32x4 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    if (nk > 0) {
        gload(kbeg);
        lstore(0);
        __syncthreads();
        for (int kt = 0; kt < nk; ++kt) {
            const int cur = kt & 1;
            if (kt + 1 < nk) gload(kbeg + (kt + 1) * BK);
            const uint16_t* sa = lds + cur * STAGE;
            const uint16_t* sb = sa + BM * BK;
#pragma unroll
            for (int s = 0; s < BK / 32; ++s) {
                const int chunk = s * 4 + (lane >> 4);
                uint4 af[MI], bfr[NJ];
#pragma unroll
                for (int i = 0; i < MI; ++i) {
                    const int r = wm * WTM + i * 16 + (lane & 15);
                    af[i] = *reinterpret_cast<const uint4*>(sa + r * BK + swz(r, chunk) * 8);
                }
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const int r = wn * WTN + j * 16 + (lane & 15);
                    bfr[j] = *reinterpret_cast<const uint4*>(sb + r * BK + swz(r, chunk) * 8);
                }
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8, bfr[j]), __builtin_bit_cast(bf16x8, af[i]),
                            acc[i][j], 0, 0, 0);
            }
            if (kt + 1 < nk) lstore(cur ^ 1);
            __syncthreads();
        }
    }

    // ---- epilogue: lane owns C[m][n..n+3] --------------------------------
    const int mrow = lane & 15, ncol = 4 * (lane >> 4);
    if constexpr (!Tr::group_k) {
        uint16_t* C = reinterpret_cast<uint16_t*>(p.c);
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const int m = wm * WTM + i * 16 + mrow;
            if (m >= rows) continue;
            const int64_t crow = (int64_t)(row0 + m) * p.ldc;
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int n = nt * BN + wn * WTN + j * 16 + ncol;
                float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
                if constexpr (KIND == GEMM_DACT) {
                    const uint2 uu = *reinterpret_cast<const uint2*>(p.u + crow + n);
                    v[0] *= dsilu_fast(bf_lo(uu.x));
                    v[1] *= dsilu_fast(bf_hi(uu.x));
                    v[2] *= dsilu_fast(bf_lo(uu.y));
                    v[3] *= dsilu_fast(bf_hi(uu.y));
                }
                *reinterpret_cast<uint2*>(C + crow + n) =
                    make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
                if constexpr (DUAL) {
                    *reinterpret_cast<uint2*>(p.c2 + crow + n) = make_uint2(
                        pack_bf2(silu_fast(v[0]), silu_fast(v[1])),
                        pack_bf2(silu_fast(v[2]), silu_fast(v[3])));
                }
            }
        }
    } else {
        float* C = p.dw[e];
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const int m = mt * BM + wm * WTM + i * 16 + mrow;
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int n = nt * BN + wn * WTN + j * 16 + ncol;
                *reinterpret_cast<f32x4*>(C + (int64_t)m * p.ldc + n) = acc[i][j];
            }
        }
    }
}

}  // namespace

hipError_t launch_gemm(GemmKind kind, bool dual, const GemmParams& p, hipStream_t s) {
    if (p.N % BN != 0) return hipErrorInvalidValue;
    dim3 block(kThreads);
    const bool group_k = kind == GEMM_DW_DOWN || kind == GEMM_DW_UP;
    int64_t grid;
    if (group_k) {
        if (p.M % BM != 0) return hipErrorInvalidValue;
        grid = (int64_t)p.E * (p.M / BM) * (p.N / BN);
    } else {
        if (p.K % BK != 0) return hipErrorInvalidValue;
        // sum_e ceil(cnt_e / BM) <= ceil(slots / BM) + E - 1
        grid = ((int64_t)(p.slots + BM - 1) / BM + p.E) * (p.N / BN);
    }
    if (grid <= 0) return hipSuccess;
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    switch (kind) {
        case GEMM_UP:
            if (dual) grouped_gemm_kernel<GEMM_UP, true><<<(unsigned)grid, block, 0, s>>>(p);
            else grouped_gemm_kernel<GEMM_UP, false><<<(unsigned)grid, block, 0, s>>>(p);
            break;
        case GEMM_DOWN: grouped_gemm_kernel<GEMM_DOWN, false><<<(unsigned)grid, block, 0, s>>>(p); break;
        case GEMM_DACT: grouped_gemm_kernel<GEMM_DACT, false><<<(unsigned)grid, block, 0, s>>>(p); break;
        case GEMM_DX: grouped_gemm_kernel<GEMM_DX, false><<<(unsigned)grid, block, 0, s>>>(p); break;
        case GEMM_DW_DOWN: grouped_gemm_kernel<GEMM_DW_DOWN, false><<<(unsigned)grid, block, 0, s>>>(p); break;
        case GEMM_DW_UP: grouped_gemm_kernel<GEMM_DW_UP, false><<<(unsigned)grid, block, 0, s>>>(p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace tmt
