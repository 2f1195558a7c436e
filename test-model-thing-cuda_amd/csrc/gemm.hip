// gemm.hip -- grouped bf16 MFMA GEMMs over expert segments (gfx950).
//
// Replaces the reference's per-expert cuBLAS loops (tmt-cuda/src/moe.cu:431-436
// forward, :533-539 backward; wrappers tmt-cuda/src/linalg.cu:9-41) and the
// gather kernel (moe.cu:127-140): one launch covers all experts, tiles are
// found from the device-side offset table (no host sync, no 128-row padding),
// and the forward token gather is folded into the operand addressing.
//
// Tile: 256 x 256 outputs per 256-thread workgroup (one workgroup per CU),
// 4 waves in 2 x 2, each wave 128 x 128 = 4 x 4 v_mfma_f32_32x32x16_bf16
// tiles (256 fp32 accumulators per lane, held in AGPRs).
//
// Operand staging: direct global -> LDS loads (global_load_lds_dwordx4, the
// data never passes through VGPRs). Two ring layouts:
//   * split rings (the activation GEMMs on 256 x 256 tiles): K = 64 tiles,
//     the A operand in a ring of 3 slots and B in a ring of 2 (32 KiB each,
//     160 KiB in all). Iteration kt loads B(kt+1) and A(kt+2). K = 64 makes
//     each K-contiguous row a full 128-byte segment: the CU accepts one
//     1 KiB load per 16 cycles when every row segment of the load is >= 128
//     bytes, but only one per 29-34 cycles with 64-byte segments from L2 or
//     HBM, so with K = 32 stages the loads alone filled the CU's load path;
//   * one ring of NST stages of K = 32 (32 KiB for 256 x 256, 24 KiB for
//     256 x 128), issued NST - 1 tiles ahead (weight-gradient GEMMs, the
//     MXFP4 variants and 128-column tiles).
//   * K-contiguous operands (activations in every GEMM, weights in the
//     forward) land as [256 rows][32] bf16, 16-byte chunks XOR-swizzled by
//     (row >> 2) & 3, and are read with ds_read_b128.
//   * Row-contiguous operands (weights read as [K][N] in the backward, and
//     the token-major operands of the weight-gradient GEMMs) land as
//     [32 k][256] bf16, chunks swizzled by 4 * (k & 3), and are read with the
//     gfx950 transposing ds_read_b64_tr_b16: inside each 16-lane group, lane
//     r points at row k0 + r/4, columns c0 + 4(r%4) .. +3, and lane i receives
//     column c0 + i of rows k0 .. k0+3 -- a K-contiguous MFMA fragment.
// The loads are issued from inline asm with explicit vmcnt accounting: the
// compiler would otherwise wait for every outstanding LDS-DMA load before
// each LDS read. Masked rows/columns are clamped to valid addresses (they
// only feed outputs that are not stored), except the reduction tail of the
// weight-gradient GEMMs, which is zeroed in LDS.
//
// Epilogue: accumulators go through LDS (fp32, 16-byte chunks swizzled by
// row) so every global store is a 16-byte vector and each output row is
// written as one contiguous 256-byte (bf16) or 512-byte (fp32) run; the
// stores (and GEMM_DACT's pre-activation reads) are non-temporal.
#include "device_util.hpp"
#include "moe_internal.hpp"

namespace tmt {
namespace {

constexpr int BM = kGemmTileRows;  // tile rows of the large-problem kernels (TBM: the tile's own)

// Tile geometry. BK_ is the K depth of one LDS stage (32 or 64), NST the
// number of stages in the ring, BN_ the tile width and NWM_ the waves along
// M (2 x NWM_ waves per workgroup):
//   BN 256, NWM 2: one 4-wave workgroup per CU, 128 x 128 wave tiles;
//   BN 256, NWM 4: one 8-wave workgroup per CU, 64 x 128 wave tiles (two
//                  waves per SIMD on the same operand tiles);
//   BN 128, NWM 2: two 4-wave workgroups per CU, 128 x 64 wave tiles, so one
//                  workgroup's waits and epilogue overlap the other's MFMAs.
template <int BK_, int NST, int BN_, int NWM_ = 2, int BM_ = 256>
struct Geo {
    static constexpr int BM = BM_;
    static constexpr int BK = BK_;
    static constexpr int NSTAGE = NST;
    static constexpr int BN = BN_;
    static constexpr int NWM = NWM_, NW = 2 * NWM_, NT = 64 * NW;  // waves, threads
    static constexpr int WTM = BM / NWM, MI = WTM / 32;  // wave tile rows
    static constexpr int WTN = BN / 2, NJ = WTN / 32;  // wave tile columns
    static constexpr int EPR = NWM == 2 ? 64 : 32;     // epilogue rows per wave and pass
    static constexpr int KCH = BK / 8;                 // 16-byte chunks per K-contiguous row
    static constexpr int OPND_A = BM * BK;             // bf16 elements of the A tile
    static constexpr int OPND_B = BN * BK;             // bf16 elements of the B tile
    static constexpr int STAGE = OPND_A + OPND_B;      // A then B
    static constexpr int DMA_A = OPND_A * 2 / 1024 / NW;  // 1 KiB wave loads per wave, A tile
    static constexpr int DMA_B = OPND_B * 2 / 1024 / NW;  // ... B tile
    static constexpr int DMA_PER_TILE = DMA_A + DMA_B;
    static constexpr int KC_ROWS = 1024 / (2 * BK);    // K-contiguous rows per wave load
    static constexpr int STEPS = BK / 16;              // MFMA k16 steps per stage
    static constexpr int WGS = BN == 256 && BM == 256 ? 1 : 2;  // workgroups per CU
    // the epilogue's fp32 staging ([EPR][WTN] per wave); the kernel sizes the
    // ring (single or split) and checks the total
    static constexpr int EPI = NW * EPR * WTN * 4;
    // K-contiguous rows: 16-byte chunk swizzle making 16 consecutive rows (the
    // lanes one ds_read_b128 cycle serves from the 64 banks = 256 bytes) hit
    // distinct banks: rows r and r + 4j share (r & 3) * 64 bytes of bank offset
    // (BK 32: 64-byte rows), so the chunk is XORed with (r >> 2) & 3; with
    // 128-byte rows (BK 64) rows r and r + 2j pair up, XOR with (r >> 1) & 7.
    static __device__ __forceinline__ int kc_swz(int r) {
        return KCH == 4 ? ((r >> 2) & 3) : ((r >> 1) & 7);
    }
    // Row-contiguous [BK][256 or 128] tiles (rows of 512 / 256 bytes, all
    // starting at bank 0): the 32 lanes of one ds_read_b64_tr_b16 cycle read
    // 4 k rows x 4 chunks; XOR with 4 * (k & 3) spreads them over 16 distinct
    // chunks (256 bytes).
    static __device__ __forceinline__ int mc_swz(int k) { return 4 * (k & 3); }
};

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

template <int KIND> struct Traits;
// C[slot][n] = X[perm[slot]] . W_up[e][n]              A: K-contig (gathered), B: K-contig
template <> struct Traits<GEMM_UP> {
    static constexpr bool group_k = false, a_kc = true, b_kc = true, gather = true, b_fp4 = false;
};
// C[slot][n] = A[slot] . W_down[e][n]
template <> struct Traits<GEMM_DOWN> {
    static constexpr bool group_k = false, a_kc = true, b_kc = true, gather = false, b_fp4 = false;
};
// C[slot][n] = (dO[slot] . W_down[e][:, n]) * silu'(U)  B: [K][N]; silu'(U) as the
// up GEMM wrote it (p.u)
template <> struct Traits<GEMM_DACT> {
    static constexpr bool group_k = false, a_kc = true, b_kc = false, gather = false, b_fp4 = false;
};
// C[slot][n] = dU[slot] . W_up[e][:, n]                 B: [K][N]
template <> struct Traits<GEMM_DX> {
    static constexpr bool group_k = false, a_kc = true, b_kc = false, gather = false, b_fp4 = false;
};
// dW_down[e][m][n] = sum_slot dO[slot][m] * A[slot][n]
template <> struct Traits<GEMM_DW_DOWN> {
    static constexpr bool group_k = true, a_kc = false, b_kc = false, b_fp4 = false;
};
// dW_up[e][m][n] = sum_slot dU[slot][m] * Xg[slot][n]   (Xg: X gathered to slot order)
template <> struct Traits<GEMM_DW_UP> {
    static constexpr bool group_k = true, a_kc = false, b_kc = false, b_fp4 = false;
};

// MXFP4 variants: same as GEMM_UP / GEMM_DOWN, B = e2m1 weights + e8m0 scales.
template <> struct Traits<GEMM_UP_FP4> {
    static constexpr bool group_k = false, a_kc = true, b_kc = true, gather = true, b_fp4 = true;
};
template <> struct Traits<GEMM_DOWN_FP4> {
    static constexpr bool group_k = false, a_kc = true, b_kc = true, gather = false, b_fp4 = true;
};

// 8 e2m1 codes (low nibble first) sharing one e8m0 scale -> 8 bf16, with the
// gfx950 scaled conversion (two codes per instruction). e2m1 values have at
// most two significant bits, so every product with 2^(scale - 127) inside
// bf16's exponent range is exact; the scale byte becomes the fp32 2^(s-127)
// (s = 0 is the subnormal 2^-127).
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 dequant8(uint32_t w, uint32_t scale) {
    const float sc = __uint_as_float(scale == 0 ? 0x00400000u : (scale << 23));
    return make_uint4(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 0)),
                      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 1)),
                      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 2)),
                      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 3)));
}

// Streaming (non-temporal) 16-byte accesses for the epilogue: outputs are
// written once and read by a later kernel, so they should not displace the
// operand tiles the other workgroups are reusing from L2.
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void st16_nt(void* p, uint4 v) {
    __builtin_nontemporal_store(u32x4_t{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4_t*>(p));
}
__device__ __forceinline__ void st16_nt(void* p, f32x4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
}
__device__ __forceinline__ uint4 ld16_nt(const uint16_t* p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// One wave-wide 16-byte-per-lane load from global memory into LDS at
// lds_base + 16 * lane (lds_base must be wave-uniform).
// M0 is written here and declared clobbered (clang warns that it is reserved).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* g, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_base) : "m0");
}
#pragma clang diagnostic pop
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N));
}

// Split-K of the last round (GEMM_DOWN / GEMM_DX, tiles 256 x BN, one
// workgroup per CU). The activation tiles are numbered expert segment by
// segment, M tile mt of all ntn column tiles; with ntn <= 8 and W resident
// workgroups, the tiles with mt < cut (cut * ntn a multiple of W) fill whole
// rounds. The R = (MT - cut) * ntn tiles left would otherwise run as one
// short round on R CUs while the rest idle, so each is cut into S parts
// along K (S = W / R, at least 8 k tiles a part). Part q of tail tile j is
// workgroup F + j*S + q (F = cut * ntn, after the whole rounds in launch
// order); it writes an fp32 partial tile, and split_fixup_kernel adds a
// tile's S partials in part order and stores the bf16 result.
struct SplitPlan {
    int cut = 0, F = 0, R = 0, S = 1, chunk = 0;  // chunk: reduction length of a part
};
template <int TBM = BM>
__device__ __forceinline__ int act_mtiles(const GemmParams& p) {
    int mt = 0;
    for (int ee = 0; ee < p.E; ++ee) mt += (p.offsets[ee + 1] - p.offsets[ee] + TBM - 1) / TBM;
    return mt;
}
template <int BK>
__device__ __forceinline__ SplitPlan split_plan(const GemmParams& p, int ntn, int mtiles) {
    SplitPlan sp;
    const int W = p.resident;
    // W a multiple of 256: the launch-order permutation of workgroups stays
    // inside aligned blocks of 256, so the first F workgroups are the rounds' tiles.
    if (p.part == nullptr || ntn > 8 || W <= 0 || W % 256 != 0 || W % ntn != 0) return sp;
    const int per = W / ntn;  // M tiles per round
    sp.cut = (mtiles / per) * per;
    sp.F = sp.cut * ntn;
    sp.R = (mtiles - sp.cut) * ntn;
    const int nk = p.K / BK;
    int S = sp.R > 0 ? W / sp.R : 1;
    S = min(S, nk / 8);
    if (S < 2) return SplitPlan{};
    sp.S = S;
    sp.chunk = ((nk + S - 1) / S) * BK;
    return sp;
}
// Expert segment of activation M tile mt (TBM rows per tile): expert, first
// slot, rows (e < 0: none).
template <int TBM = BM>
__device__ __forceinline__ void act_tile(const GemmParams& p, int mt, int& e, int& row0, int& rows) {
    e = -1;
    int t0 = 0;
    for (int ee = 0; ee < p.E; ++ee) {
        const int beg = p.offsets[ee], end = p.offsets[ee + 1];
        const int tiles = (end - beg + TBM - 1) / TBM;
        if (mt < t0 + tiles) {
            e = ee;
            row0 = beg + (mt - t0) * TBM;
            rows = min(TBM, end - row0);
            return;
        }
        t0 += tiles;
    }
}

// Split rings (A in NST slots, B in NST - 1) for K = 64 tiles of the
// activation GEMMs on 256 x 256 tiles.
template <int KIND, int BK, int BN, int NWM, int TBM = BM>
constexpr bool split_ring() {
    return BK == 64 && BN == 256 && NWM == 2 && TBM == 256 && !Traits<KIND>::group_k;
}

// Persistent kernels: the split-ring GEMMs (every tile of a launch has the
// same K, so a static schedule stays balanced) run one workgroup per CU that
// walks the tiles vb = blockIdx.x, blockIdx.x + gridDim.x, ... . A tile's
// first operand loads then go out while the previous tile's epilogue stores
// drain, and the per-workgroup launch and set-up cost is paid once per CU
// instead of once per tile. vb keeps the launch-order meaning of blockIdx.x
// (gridDim.x is a multiple of 8 whenever it is below the tile count, so vb
// runs on XCD vb % 8 as the tile map assumes).
template <int KIND, int BK, int BN, int NWM, int TBM = BM>
constexpr bool persistent_tiles() {
    return split_ring<KIND, BK, BN, NWM, TBM>();
}

// LDS of one workgroup: the operand ring, or the epilogue's fp32 staging if
// larger (MXFP4 B operand per stage: 256 rows x BK/2 bytes of codes, then
// one 1 KiB copy per wave of the row scales).
template <int KIND, int BK_, int NST, int BN_, int NWM_, int BM_>
constexpr int gemm_lds_bytes() {
    using Gm = Geo<BK_, NST, BN_, NWM_, BM_>;
    constexpr int codes = 256 * (BK_ / 2), scales = 4 * 1024;
    constexpr int stage = Traits<KIND>::b_fp4 ? Gm::OPND_A + (codes + scales) / 2 : Gm::STAGE;
    constexpr int bslot = Traits<KIND>::b_fp4 ? (codes + scales) / 2 : Gm::OPND_B;
    constexpr int ring = split_ring<KIND, BK_, BN_, NWM_, BM_>() ? (NST * Gm::OPND_A + (NST - 1) * bslot) * 2
                                                                : NST * stage * 2;
    return ring > Gm::EPI ? ring : Gm::EPI;
}

// One output tile (or split-K part) of the grouped GEMM: launch-order block
// index vb; returns without touching memory when vb maps to no tile. et: the
// experts' activation tiles (unused by the weight-gradient kinds). lds_raw:
// the workgroup's gemm_lds_bytes() of LDS, declared by the kernel (measured:
// DOWN and DX about 1% faster at c3 than with the array declared here).
template <int KIND, bool DUAL, int BK_, int NST, int BN_, int NWM_ = 2, int BM_ = 256>
__device__ __forceinline__ void grouped_gemm_tile(const GemmParams& p, const int vb, const ExpertTiles& et,
                                                  uint4* lds_raw) {
    using Tr = Traits<KIND>;
    using Gm = Geo<BK_, NST, BN_, NWM_, BM_>;
    constexpr int BM = Gm::BM;
    constexpr int BK = Gm::BK, NSTAGE = Gm::NSTAGE, BN = Gm::BN, WTN = Gm::WTN, NJ = Gm::NJ;
    constexpr int WTM = Gm::WTM, MI = Gm::MI, NT = Gm::NT, EPR = Gm::EPR;
    constexpr int OPND_A = Gm::OPND_A, OPND_B = Gm::OPND_B;
    constexpr int DMA_A = Gm::DMA_A, DMA_B = Gm::DMA_B;
    constexpr bool kSplit = split_ring<KIND, BK_, BN_, NWM_, BM_>();
    static_assert(!kSplit || NST == 3, "split rings: 3 A slots and 2 B slots");
    static_assert(BM == 256 || (BN == 128 && NWM_ == 2 && !Tr::b_fp4), "128-row tiles: 128 columns, 4 waves, bf16");
    // MXFP4 B operand per tile: 256 rows x BK/2 bytes of codes, then one 1 KiB
    // copy per wave of the tile's row scales (one 32-block at BK = 32, two at
    // BK = 64: lanes 16-31 load the second block's).
    static_assert(!Tr::b_fp4 || (BN == 256 && NWM_ == 2 && (BK == 32 || kSplit)), "MXFP4 tiles: 256 columns, 4 waves");
    constexpr int FP4_CODES = 256 * (BK / 2), FP4_SCALES = 4 * 1024;
    constexpr int STAGE = Tr::b_fp4 ? OPND_A + (FP4_CODES + FP4_SCALES) / 2 : Gm::STAGE;  // bf16 elements
    constexpr int DMA_PER_TILE = Tr::b_fp4 ? DMA_A + 2 : Gm::DMA_PER_TILE;
    // split rings: B slot size (bf16 elements) and wave loads per B tile
    constexpr int B_SLOT = Tr::b_fp4 ? (FP4_CODES + FP4_SCALES) / 2 : OPND_B;
    constexpr int DMA_BT = Tr::b_fp4 ? FP4_CODES / 1024 / 4 + 1 : DMA_B;
    constexpr int KCH = Gm::KCH, KC_ROWS = Gm::KC_ROWS, STEPS = Gm::STEPS;
    constexpr int RING = kSplit ? (NST * OPND_A + (NST - 1) * B_SLOT) * 2 : NSTAGE * STAGE * 2;
    constexpr int LDS_TOTAL = RING > Gm::EPI ? RING : Gm::EPI;
    static_assert(LDS_TOTAL * Gm::WGS <= 160 * 1024, "LDS ring too large");
    static_assert(LDS_TOTAL == gemm_lds_bytes<KIND, BK_, NST, BN_, NWM_, BM_>(), "LDS size of the kernel's array");
    uint16_t* lds = reinterpret_cast<uint16_t*>(lds_raw);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    // the wave's first row and column in the tile
    const int wrow = (wave >> 1) * WTM, wcol = (wave & 1) * WTN;
    const int ntn = (p.N + BN - 1) / BN;

    // ---- tile coordinates -------------------------------------------------
    // The hardware hands workgroup b to XCD b % 8 and each XCD runs 32 at a
    // time (one per CU). Workgroups b = 8j + x with j in [32t, 32t + 32) are
    // therefore co-resident on XCD x; they get the 32 tiles of group
    // G = 8t + x, laid out as gm x gn tiles (gn = min(tiles across N, 8)) so
    // that the XCD's L2 serves each operand slice to several workgroups.
    // Consecutive groups go to different XCDs, which spreads the long tiles
    // of the weight-gradient GEMMs (experts in descending-count order).
    const int lid = (((vb >> 8) << 3) + (vb & 7)) * 32 + ((vb >> 3) & 31);
    const int G = lid >> 5, gi = lid & 31;
    const int gn = min(ntn, 8), gm = 32 / gn;
    const int ngn = (ntn + gn - 1) / gn;
    int e = -1, mt = 0, nt = 0;
    int row0 = 0, rows = 0;   // activation GEMMs: slot range of this tile
    int kbeg = 0, kend = 0;   // reduction range (slots for dW GEMMs)
    int mlim = 0;             // valid output rows in this tile
    constexpr bool kSplitK = (KIND == GEMM_DOWN || KIND == GEMM_DX) && BM == 256;
    int part_unit = -1;  // split-K tail: index of this workgroup's partial tile
    if constexpr (!Tr::group_k) {
        kbeg = 0;
        kend = p.K;
        SplitPlan sp;
        if constexpr (kSplitK) {
            if (p.part != nullptr) sp = split_plan<BK>(p, ntn, et.total);
        }
        if (p.xcd_runs) {
            // Launches whose tiles all run at once: the tiles in (mt, nt)
            // order, nt fastest, cut into 8 runs of `per`; workgroup vb runs
            // on XCD vb % 8 and takes tile vb / 8 of that XCD's run. Every
            // XCD gets the same number of tiles, and a run covers whole rows
            // of tiles of one or two experts, whose weights its L2 keeps.
            const int R = et.total * ntn;
            const int per = (R + 7) / 8;
            const int j = (vb & 7) * per + (vb >> 3);
            if ((vb >> 3) >= per || j >= R) return;
            mt = j / ntn;
            nt = j - mt * ntn;
        } else if (sp.S >= 2 && vb >= sp.F) {
            const int u = vb - sp.F;
            if (u >= sp.R * sp.S) return;
            const int j = u / sp.S, q = u - j * sp.S;
            mt = sp.cut + j / ntn;
            nt = j % ntn;
            kbeg = q * sp.chunk;
            kend = min(p.K, kbeg + sp.chunk);
            part_unit = u;
        } else {
            if (gi >= gm * gn) return;
            mt = (G / ngn) * gm + gi % gm;
            nt = (G % ngn) * gn + gi / gm;
            if (nt >= ntn) return;
        }
        if (!expert_tile<BM>(et, mt, e, row0, rows)) return;  // beyond the last tile of the last expert
        mlim = rows;
    } else {
        // A group's work is proportional to its expert's count, and groups
        // come in descending-count order. With G % 8 as the XCD, an expert
        // whose groups fill half of the XCDs sends every following expert to
        // the same halves in turn (c3: 74K against 57K slots per XCD).
        //  * 128-column tiles (two workgroups per CU): round r hands its 8
        //    groups of 32 tiles to the XCDs in snake order (reversed on odd
        //    rounds), which keeps every XCD's sum of counts near the mean;
        //  * 256-column tiles (one per CU): groups of 16 tiles, two per XCD
        //    and round, paired heaviest with lightest (XCD x runs groups
        //    16r + x and 16r + 15 - x). With 32-tile groups the XCD holding
        //    the heaviest expert's group could not be balanced.
        constexpr int GSZ = BN == 256 ? 16 : 32;
        const int rnd = vb >> 8, xcd = vb & 7, sub = (vb >> 3) & 31;
        const int Gs = GSZ == 16 ? 16 * rnd + (sub < 16 ? xcd : 15 - xcd) : 8 * rnd + ((rnd & 1) ? 7 - xcd : xcd);
        const int gk = sub & (GSZ - 1), gnk = min(ntn, 8), gmk = GSZ / gnk, ngnk = (ntn + gnk - 1) / gnk;
        if (gk >= gmk * gnk) return;
        const int ntm = (p.M + BM - 1) / BM;
        const int gpe = ((ntm + gmk - 1) / gmk) * ngnk;  // groups per expert
        const int ei = Gs / gpe, g = Gs - ei * gpe;
        if (ei >= p.E) return;
        mt = (g / ngnk) * gmk + gk % gmk;
        nt = (g % ngnk) * gnk + gk / gmk;
        if (mt >= ntm || nt >= ntn) return;
        e = p.order[ei];
        kbeg = p.offsets[e];
        kend = p.offsets[e + 1];
        mlim = min(BM, p.M - mt * BM);
    }
    const int col0 = nt * BN;                // the tile's first output column
    const int nlim = min(BN, p.N - col0);  // valid output columns in this tile
    const int nk = (kend - kbeg + BK - 1) / BK;

    // ---- DMA addressing -----------------------------------------------------
    // K-contiguous tile: wave load q covers rows KC_ROWS*q .. +KC_ROWS-1;
    // lane -> row KC_ROWS*q + lane/KCH, physical chunk lane%KCH, logical chunk
    // (lane%KCH) ^ kc_swz(row). Row-contiguous tile of C chunks per k row
    // (32 for 256 columns, 16 for 128): wave load q covers k rows
    // (64/C)q .. ; lane -> k = (64/C)q + lane/C, physical chunk lane%C,
    // logical chunk (lane%C) ^ mc_swz(k).
    // K-contiguous operands keep one source pointer per wave load; row-
    // contiguous ones keep a column pointer and the lane's k row, clamped to
    // the last valid reduction index when issued (the tail is zeroed in LDS).
    const uint16_t* a_ptr[DMA_A];
    const uint16_t* b_ptr[DMA_B];
    int a_k[DMA_A], b_k[DMA_B];
#pragma unroll
    for (int i = 0; i < DMA_A; ++i) {
        const int q = wave * DMA_A + i;
        if constexpr (Tr::a_kc) {
            const int r = KC_ROWS * q + lane / KCH;
            const int c = (lane % KCH) ^ Gm::kc_swz(r);
            const int slot = min(row0 + r, p.slots - 1);
            const int src = Tr::gather ? p.perm[slot] : slot;
            a_ptr[i] = p.a + (int64_t)src * p.lda + c * 8;
            a_k[i] = 0;
        } else {
            constexpr int C = BM / 8;  // 16-byte chunks per k row
            const int k = (64 / C) * q + lane / C;
            const int c = (lane % C) ^ Gm::mc_swz(k);
            a_ptr[i] = p.a + min(mt * BM + c * 8, p.M - 8);
            a_k[i] = k;
        }
    }
#pragma unroll
    for (int i = 0; i < DMA_B; ++i) {
        const int q = wave * DMA_B + i;
        if constexpr (Tr::b_fp4) {
            b_ptr[i] = nullptr;
            b_k[i] = 0;
        } else if constexpr (Tr::b_kc) {
            const int r = KC_ROWS * q + lane / KCH;
            const int c = (lane % KCH) ^ Gm::kc_swz(r);
            const int n = min(col0 + r, p.N - 1);
            b_ptr[i] = p.w[e] + (int64_t)n * p.ldb + c * 8;
            b_k[i] = 0;
        } else {
            constexpr int C = BN / 8;
            const int k = (64 / C) * q + lane / C;
            const int c = (lane % C) ^ Gm::mc_swz(k);
            const uint16_t* base = Tr::group_k ? p.b : p.w[e];
            b_ptr[i] = base + min(col0 + c * 8, p.N - 8);
            b_k[i] = k;
        }
    }
    // MXFP4: wave w loads the codes of rows 64w + lane (16 bytes per tile) and
    // its own copy of the tile's 256 row scales (lane l -> rows 16(l%16)..+15;
    // row groups past N are clamped to the tile's first group).
    // With split rings (BK = 64) lane pair (2m, 2m+1) loads the 32 code bytes
    // of row m (two 16-byte halves, swapped in LDS when bit 3 of m is set) and
    // lanes 16-31 load the second scale block.
    const uint8_t* q_ptr = nullptr;
    const uint8_t* q2_ptr[2] = {nullptr, nullptr};
    const uint8_t* sc_ptr = nullptr;
    if constexpr (Tr::b_fp4) {
        const int g = nt * BN + 16 * (lane & 15);
        if constexpr (kSplit) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int sl = (wave * 2 + i) * 64 + lane, m = sl >> 1;
                const int half = (sl & 1) ^ ((m >> 3) & 1);
                q2_ptr[i] = p.wq[e] + (int64_t)min(nt * BN + m, p.N - 1) * (p.K / 2) + half * 16;
            }
            sc_ptr = p.wsc[e] + (int64_t)((lane >> 4) & 1) * p.N + (g < p.N ? g : nt * BN);
        } else {
            const int n = min(nt * BN + 64 * wave + lane, p.N - 1);
            q_ptr = p.wq[e] + (int64_t)n * (p.K / 2);
            sc_ptr = p.wsc[e] + (g < p.N ? g : nt * BN);
        }
    }
    const uint32_t lds0 = lds_addr(lds);
    // bf16 element offsets of tile t's A and B operand tiles in LDS
    auto a_slot = [&](int t) -> int { return kSplit ? (t % NST) * OPND_A : (t % NSTAGE) * STAGE; };
    auto b_slot = [&](int t) -> int {
        return kSplit ? NST * OPND_A + (t % (NST - 1)) * B_SLOT : (t % NSTAGE) * STAGE + OPND_A;
    };
    // Wave load i of tile t's A / B operand (t clamped to the last real tile
    // so the per-tile load count stays constant).
    auto dma_a = [&](int t, int i) {
        const int k0 = kbeg + min(t, nk - 1) * BK;
        const uint16_t* ga = Tr::a_kc ? a_ptr[i] + k0 : a_ptr[i] + (int64_t)min(k0 + a_k[i], kend - 1) * p.lda;
        dma16(ga, lds0 + (uint32_t)a_slot(t) * 2u + (uint32_t)(wave * DMA_A + i) * 1024u);
    };
    auto dma_b = [&](int t, int i) {
        const int k0 = kbeg + min(t, nk - 1) * BK;
        if constexpr (Tr::b_fp4) {
            const uint32_t sb = lds0 + (uint32_t)b_slot(t) * 2u;
            if (i < DMA_BT - 1) dma16(q2_ptr[i] + k0 / 2, sb + (uint32_t)(wave * (DMA_BT - 1) + i) * 1024u);
            else dma16(sc_ptr + (int64_t)(k0 / 32) * p.N, sb + FP4_CODES + (uint32_t)wave * 1024u);
        } else {
            const uint16_t* gb = Tr::b_kc ? b_ptr[i] + k0 : b_ptr[i] + (int64_t)min(k0 + b_k[i], kend - 1) * p.ldb;
            dma16(gb, lds0 + (uint32_t)b_slot(t) * 2u + (uint32_t)(wave * DMA_B + i) * 1024u);
        }
    };
    // Issue the 8 wave loads of K tile t (clamped to the last real tile so the
    // per-tile load count stays constant) into stage t % NSTAGE.
    auto dma_tile = [&](int t) {
        const int k0 = kbeg + min(t, nk - 1) * BK;  // first reduction index of the tile
        const uint32_t sbase = lds0 + (uint32_t)((t % NSTAGE) * STAGE) * 2u;
#pragma unroll
        for (int i = 0; i < DMA_A; ++i) {
            const uint32_t qoff = (uint32_t)(wave * DMA_A + i) * 1024u;
            const uint16_t* ga = Tr::a_kc ? a_ptr[i] + k0
                                          : a_ptr[i] + (int64_t)min(k0 + a_k[i], kend - 1) * p.lda;
            dma16(ga, sbase + qoff);
        }
        if constexpr (!Tr::b_fp4) {
#pragma unroll
            for (int i = 0; i < DMA_B; ++i) {
                const uint32_t qoff = (uint32_t)(wave * DMA_B + i) * 1024u;
                const uint16_t* gb = Tr::b_kc ? b_ptr[i] + k0
                                              : b_ptr[i] + (int64_t)min(k0 + b_k[i], kend - 1) * p.ldb;
                dma16(gb, sbase + OPND_A * 2u + qoff);
            }
        } else {
            const int kb = k0 / 32;  // scale block of this tile
            dma16(q_ptr + kb * 16, sbase + OPND_A * 2u + (uint32_t)wave * 1024u);
            dma16(sc_ptr + (int64_t)kb * p.N, sbase + OPND_A * 2u + FP4_CODES + (uint32_t)wave * 1024u);
        }
    };
    // Load `idx` of dma_tile(t) on its own, for interleaving with the MFMAs.
    auto dma_one = [&](int t, int idx) {
        const int k0 = kbeg + min(t, nk - 1) * BK;
        const uint32_t sbase = lds0 + (uint32_t)((t % NSTAGE) * STAGE) * 2u;
        if (idx < DMA_A) {
            const uint32_t qoff = (uint32_t)(wave * DMA_A + idx) * 1024u;
            const uint16_t* ga = Tr::a_kc ? a_ptr[idx] + k0
                                          : a_ptr[idx] + (int64_t)min(k0 + a_k[idx], kend - 1) * p.lda;
            dma16(ga, sbase + qoff);
        } else {
            const int i = idx - DMA_A;
            const uint32_t qoff = (uint32_t)(wave * DMA_B + i) * 1024u;
            const uint16_t* gb = Tr::b_kc ? b_ptr[i] + k0
                                          : b_ptr[i] + (int64_t)min(k0 + b_k[i], kend - 1) * p.ldb;
            dma16(gb, sbase + OPND_A * 2u + qoff);
        }
    };
    // Reduction tail of the weight-gradient GEMMs: zero k rows >= kvalid of
    // the last tile in both operand tiles (rows of 512 bytes).
    auto zero_tail = [&](int t) {
        if constexpr (Tr::group_k) {
            const int kvalid = kend - (kbeg + t * BK);
            if (kvalid < BK) {
                uint16_t* st = lds + (t % NSTAGE) * STAGE;
                const int na = (BK - kvalid) * (BM / 8), nb = (BK - kvalid) * (BN / 8);  // 16-byte vectors
                for (int v = tid; v < na + nb; v += NT) {
                    if (v < na) *reinterpret_cast<uint4*>(st + kvalid * BM + v * 8) = make_uint4(0, 0, 0, 0);
                    else *reinterpret_cast<uint4*>(st + OPND_A + kvalid * BN + (v - na) * 8) = make_uint4(0, 0, 0, 0);
                }
            }
        }
    };

    // ---- fragments ----------------------------------------------------------
    struct Frag {
        uint4 a[MI], b[NJ];
    };
    // K-contiguous: lane reads row base + lane%32, chunk 2s + lane/32.
    auto read_kc = [&](const uint16_t* t, int rbase, int s) {
        const int r = rbase + (lane & 31);
        const int c = (2 * s + (lane >> 5)) ^ Gm::kc_swz(r);
        return *reinterpret_cast<const uint4*>(t + r * BK + c * 8);
    };
    // Row-contiguous: two transposing reads give k = 16s + 8(lane/32) + 0..7
    // for column cbase + lane%32.
    auto read_mc = [&](const uint16_t* t, int stride, int cbase, int s) {
        const int g = lane >> 4, r = lane & 15;
        const int col = cbase + 16 * (g & 1) + 4 * (r & 3);
        const int kb = 16 * s + 8 * (g >> 1) + (r >> 2);
        uint32_t w[4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int k = kb + 4 * h;
            const int c = (col >> 3) ^ Gm::mc_swz(k);
            const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s16x4*)(t + k * stride + c * 8 + (col & 7)));
            w[2 * h] = (uint32_t)(uint16_t)v[0] | ((uint32_t)(uint16_t)v[1] << 16);
            w[2 * h + 1] = (uint32_t)(uint16_t)v[2] | ((uint32_t)(uint16_t)v[3] << 16);
        }
        return make_uint4(w[0], w[1], w[2], w[3]);
    };
    // MXFP4: lane reads 4 bytes (8 codes: k = 16s + 8(lane/32) .. +7) of row
    // rbase + lane%32 and that row's scale from its wave's copy, and expands
    // them to a bf16 fragment.
    auto read_fp4 = [&](const uint16_t* tB, int rbase, int s) {
        const uint8_t* codes = reinterpret_cast<const uint8_t*>(tB);
        const uint8_t* scales = codes + FP4_CODES + wave * 1024;
        const int r = rbase + (lane & 31);
        if constexpr (kSplit) {
            // k = 16s + 8(lane/32) .. +7: byte 8s + 4(lane/32) of the row's 32
            const int blk = s >> 1, within = (8 * s + 4 * (lane >> 5)) & 15;
            const uint32_t w = *reinterpret_cast<const uint32_t*>(
                codes + r * 32 + ((blk ^ ((lane >> 3) & 1)) * 16) + within);
            return dequant8(w, scales[blk * 256 + r]);
        } else {
            const uint32_t w = *reinterpret_cast<const uint32_t*>(codes + r * 16 + (2 * s + (lane >> 5)) * 4);
            return dequant8(w, scales[r]);
        }
    };
    auto load_frag = [&](Frag& f, int t, int s) {
        const uint16_t* tA = lds + a_slot(t);
        const uint16_t* tB = lds + b_slot(t);
#pragma unroll
        for (int i = 0; i < MI; ++i)
            f.a[i] = Tr::a_kc ? read_kc(tA, wrow + 32 * i, s) : read_mc(tA, BM, wrow + 32 * i, s);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
            f.b[j] = Tr::b_fp4 ? read_fp4(tB, wcol + 32 * j, s)
                               : (Tr::b_kc ? read_kc(tB, wcol + 32 * j, s) : read_mc(tB, BN, wcol + 32 * j, s));
    };

    f32x16 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    // The first k16 step of a tile with the loads of tile t spread over its
    // MFMAs (one after every MI*NJ / DMA_PER_TILE of them). A wave that issues
    // the eight loads back to back leaves its SIMD's MFMA unit idle while
    // they issue. Measured on the c3 shapes: DOWN 1.115 -> 1.070 ms, UP and
    // DACT about 0.5% faster; DX (+6.6%) and the weight-gradient GEMMs
    // (+1-2.5%) keep the loads in one batch.
    constexpr bool kSpreadDma = !Tr::b_fp4 && (KIND == GEMM_DOWN || KIND == GEMM_UP || KIND == GEMM_DACT);
    auto mma_dma = [&](const Frag& f, int t) {
        constexpr int NM = MI * NJ;
        int dq = 0;
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    __builtin_bit_cast(bf16x8, f.b[j]), __builtin_bit_cast(bf16x8, f.a[i]),
                    acc[i][j], 0, 0, 0);
                const int q = i * NJ + j;
                if (dq < DMA_PER_TILE && (q + 1) * DMA_PER_TILE >= (dq + 1) * NM) {
                    __builtin_amdgcn_sched_barrier(0);
                    dma_one(t, dq);
                    __builtin_amdgcn_sched_barrier(0);
                    ++dq;
                }
            }
        for (; dq < DMA_PER_TILE; ++dq) dma_one(t, dq);
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

    // ---- main loop ----------------------------------------------------------
    // Iteration kt runs the STEPS k16 steps of tile kt. Every step first reads
    // the next step's fragments; the first step also issues the loads of
    // tile kt + NSTAGE - 1. Before the last step the wave waits for its loads
    // of tile kt+1 and the workgroup synchronises (all loads of tile kt+1 are
    // visible, and every wave is done reading the stage that the next
    // iteration refills); the last step then prefetches step 0 of tile kt+1.
    constexpr int VM_AHEAD = (NSTAGE - 2) * DMA_PER_TILE;
    if constexpr (kSplit) {
        // Split rings. Iteration kt multiplies tile kt in STEPS k16 steps;
        // the loads of B(kt+1) and then A(kt+2) are spread over the MFMAs of
        // the first STEPS - 1 steps (their slots were last read by tile kt-1,
        // before the previous barrier). Loads complete in issue order, so
        // waiting until only A(kt+2)'s loads are outstanding leaves all of
        // tile kt+1 in LDS at the barrier; the last step then prefetches
        // tile kt+1's first fragments.
        constexpr int ND = DMA_A + DMA_BT;
        auto mma_loads = [&](const Frag& f, int kt, int d0, int dn) {
            constexpr int NM = MI * NJ;
            int dq = 0;
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(bf16x8, f.b[j]), __builtin_bit_cast(bf16x8, f.a[i]),
                        acc[i][j], 0, 0, 0);
                    const int q = i * NJ + j;
                    if (dq < dn && (q + 1) * dn >= (dq + 1) * NM) {
                        const int d = d0 + dq;
                        __builtin_amdgcn_sched_barrier(0);
                        if (d < DMA_BT) dma_b(kt + 1, d);
                        else dma_a(kt + 2, d - DMA_BT);
                        __builtin_amdgcn_sched_barrier(0);
                        ++dq;
                    }
                }
        };
        auto dfirst = [](int s) { return s * ND / (STEPS - 1); };
        if (nk > 0) {
#pragma unroll
            for (int i = 0; i < DMA_A; ++i) dma_a(0, i);
#pragma unroll
            for (int i = 0; i < DMA_BT; ++i) dma_b(0, i);
#pragma unroll
            for (int i = 0; i < DMA_A; ++i) dma_a(1, i);
            wait_vm<DMA_A>();
            __syncthreads();
            Frag f[2];
            load_frag(f[0], 0, 0);
            for (int kt = 0; kt < nk; ++kt) {
#pragma unroll
                for (int s = 0; s < STEPS - 1; ++s) {
                    load_frag(f[(s + 1) & 1], kt, s + 1);
                    mma_loads(f[s & 1], kt, dfirst(s), dfirst(s + 1) - dfirst(s));
                }
                wait_vm<DMA_A>();
                __syncthreads();
                load_frag(f[0], min(kt + 1, nk - 1), 0);
                mma(f[(STEPS - 1) & 1]);
#pragma unroll
                for (int q = 0; q < MI * NJ / 2; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);  // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);  // DS read
                }
                __builtin_amdgcn_sched_group_barrier(0x008, MI * NJ / 2, 1);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else if (nk > 0) {
#pragma unroll
        for (int t = 0; t < NSTAGE - 1; ++t) dma_tile(t);
        wait_vm<(NSTAGE >= 2 ? VM_AHEAD : 0)>();
        __syncthreads();
        if (nk == 1) {
            zero_tail(0);
            __syncthreads();
        }
        Frag f[2];
        load_frag(f[0], 0, 0);
        for (int kt = 0; kt < nk; ++kt) {
#pragma unroll
            for (int s = 0; s < STEPS - 1; ++s) {
                load_frag(f[(s + 1) & 1], kt, s + 1);
                if constexpr (kSpreadDma) {
                    if (s == 0) {
                        mma_dma(f[0], kt + NSTAGE - 1);
                        continue;
                    }
                } else {
                    if (s == 0) dma_tile(kt + NSTAGE - 1);
                }
                mma(f[s & 1]);
#pragma unroll
                for (int q = 0; q < MI * NJ / 2; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
                }
                __builtin_amdgcn_sched_group_barrier(0x008, MI * NJ / 2, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
            if constexpr (NSTAGE == 2) {
                wait_vm<0>();
            } else {
                wait_vm<VM_AHEAD>();
            }
            __syncthreads();
            if (kt + 1 == nk - 1) {
                zero_tail(kt + 1);
                __syncthreads();
            }
            load_frag(f[0], min(kt + 1, nk - 1), 0);
            mma(f[1]);
#pragma unroll
            for (int q = 0; q < MI * NJ / 2; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);  // DS read
            }
            __builtin_amdgcn_sched_group_barrier(0x008, MI * NJ / 2, 1);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    wait_vm<0>();
    __syncthreads();

    // ---- epilogue ---------------------------------------------------------
    // acc[i][j][r] = C[m][n] with m = wrow + 32i + (lane&31) and
    // n = wcol + 32j + 8(r>>2) + 4(lane>>5) + (r&3) (n from the tile's col0).
    // Passes of EPR rows per wave go through an fp32 LDS region ([EPR][WTN],
    // 16-byte chunks swizzled by row), then leave as row-contiguous 16-byte
    // stores.
    constexpr int CH = WTN / 4;              // 16-byte fp32 chunks per staged row
    constexpr int LPR = WTN / 8, RPI = 64 / LPR;     // bf16 out: lanes per row, rows per instruction
    constexpr int FLPR = WTN / 4, FRPI = 64 / FLPR;  // fp32 out
    constexpr int FPP = EPR / 32, PASSES = MI / FPP;  // row fragments per pass, passes
    float* stage_f = reinterpret_cast<float*>(lds_raw) + wave * (EPR * WTN);
    const int mbase = wrow, nbase = wcol;
    // GEMM_DACT: silu'(U) of every pass is requested here, in one batch, so
    // the tile waits for one memory round trip instead of one per pass (the
    // mainloop's operand fragments are dead, which leaves room).
    constexpr int UPP = KIND == GEMM_DACT ? EPR / RPI : 1;  // U loads per lane and pass
    uint4 uin[KIND == GEMM_DACT ? PASSES : 1][UPP];
    if constexpr (KIND == GEMM_DACT && !Tr::group_k) {
        const int n = nbase + (lane % LPR) * 8;
#pragma unroll
        for (int pass = 0; pass < PASSES; ++pass)
#pragma unroll
            for (int k = 0; k < UPP; ++k) {
                const int m = mbase + pass * EPR + lane / LPR + RPI * k;
                const bool ok = m < mlim && n < nlim;
                const int64_t off = (int64_t)(row0 + (ok ? m : 0)) * p.ldc + col0 + (ok ? n : 0);
                uin[pass][k] = ld16_nt(p.u + off);
            }
    }
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) {
#pragma unroll
        for (int ii = 0; ii < FPP; ++ii) {
            const int i = pass * FPP + ii;
            const int lr = ii * 32 + (lane & 31);
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int ch = j * 8 + 2 * q + (lane >> 5);
                    *reinterpret_cast<f32x4*>(stage_f + lr * WTN + ((ch ^ (lr & (CH - 1))) * 4)) =
                        f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                              acc[i][j][4 * q + 3]};
                }
        }
        __syncthreads();
        if (kSplitK && part_unit >= 0) {
            // split-K part: the fp32 partial tile [BM][BN], rows < mlim, with
            // plain stores (split_fixup_kernel reads it right after, from
            // the caches; non-temporal stores measured 0.015 ms slower per GEMM)
            float* C = p.part + (int64_t)part_unit * BM * BN;
            const int cl = lane % FLPR;
#pragma unroll 4
            for (int rr = lane / FLPR; rr < EPR; rr += FRPI) {
                const int m = mbase + pass * EPR + rr;
                const int n = nbase + cl * 4;
                if (m >= mlim || n >= nlim) continue;
                const f32x4 v = *reinterpret_cast<const f32x4*>(stage_f + rr * WTN + ((cl ^ (rr & (CH - 1))) * 4));
                *reinterpret_cast<f32x4*>(C + (int64_t)m * BN + n) = v;
            }
        } else if constexpr (!Tr::group_k) {
            // LPR lanes per row (8 bf16 each), RPI rows per instruction
            uint16_t* C = reinterpret_cast<uint16_t*>(p.c);
            const int cl = lane % LPR;
            const int n = nbase + cl * 8;
            // element offset of the lane's first row in this pass, advanced by
            // RPI rows per store (no 64-bit multiply per store)
            const int64_t off0 = (int64_t)(row0 + mbase + pass * EPR + lane / LPR) * p.ldc + col0 + n;
            const int64_t rstep = (int64_t)RPI * p.ldc;
#pragma unroll
            for (int k = 0; k < EPR / RPI; ++k) {
                const int rr = lane / LPR + RPI * k;
                const int m = mbase + pass * EPR + rr;
                if (m >= mlim || n >= nlim) continue;
                const float* src = stage_f + rr * WTN;
                const f32x4 v0 = *reinterpret_cast<const f32x4*>(src + (((2 * cl) ^ (rr & (CH - 1))) * 4));
                const f32x4 v1 = *reinterpret_cast<const f32x4*>(src + (((2 * cl + 1) ^ (rr & (CH - 1))) * 4));
                float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                const int64_t off = off0 + k * rstep;
                if constexpr (DUAL) {
                    // U itself is not kept: C = silu'(U) (skipped when C is
                    // null, for forward-only handles), c2 = SiLU(U)
                    float a[8], da[8];
#pragma unroll
                    for (int t = 0; t < 8; ++t) silu_dsilu(v[t], a[t], da[t]);
                    if (C != nullptr) st16_nt(C + off, pack8(da));
                    st16_nt(p.c2 + off, pack8(a));
                } else {
                    if constexpr (KIND == GEMM_DACT) {
                        float ds[8];
                        unpack8(uin[pass][k], ds);  // silu'(U) from the up GEMM
#pragma unroll
                        for (int t = 0; t < 8; ++t) v[t] *= ds[t];
                    }
                    st16_nt(C + off, pack8(v));
                }
            }
        } else {
            // FLPR lanes per row (4 fp32 each), FRPI rows per instruction
            float* C = p.dw[e];
            const int cl = lane % FLPR;
#pragma unroll 4
            for (int rr = lane / FLPR; rr < EPR; rr += FRPI) {
                const int m = mbase + pass * EPR + rr;
                const int n = nbase + cl * 4;
                if (m >= mlim || n >= nlim) continue;
                const f32x4 v = *reinterpret_cast<const f32x4*>(stage_f + rr * WTN + ((cl ^ (rr & (CH - 1))) * 4));
                st16_nt(C + (int64_t)(mt * BM + m) * p.ldc + col0 + n, v);
            }
        }
        __syncthreads();
    }
}

template <int KIND, bool DUAL, int BK_, int NST, int BN_, int NWM_ = 2, int BM_ = 256>
__global__ __launch_bounds__(128 * NWM_, (BN_ == 256 && BM_ == 256 ? 1 : 2)) void grouped_gemm_kernel(GemmParams p) {
    __shared__ uint4 lds_raw[gemm_lds_bytes<KIND, BK_, NST, BN_, NWM_, BM_>() / 16];
    // the experts' tiles, once per workgroup (before any tile's stores, so
    // the vector load of the offsets waits on nothing else)
    ExpertTiles et{};
    if constexpr (!Traits<KIND>::group_k) et = expert_tiles<Geo<BK_, NST, BN_, NWM_, BM_>::BM>(p.offsets, p.E, threadIdx.x & 63);
    if constexpr (persistent_tiles<KIND, BK_, BN_, NWM_, BM_>()) {
        for (int vb = blockIdx.x; vb < p.vblocks; vb += gridDim.x)
            grouped_gemm_tile<KIND, DUAL, BK_, NST, BN_, NWM_, BM_>(p, vb, et, lds_raw);
    } else {
        grouped_gemm_tile<KIND, DUAL, BK_, NST, BN_, NWM_, BM_>(p, blockIdx.x, et, lds_raw);
    }
}

// The split-K tail's second pass: tail tile j is the sum of its S partials
// in part order, rounded once to bf16. Work items are (tile, 8-row slab);
// thread t adds 8 columns of one row.
template <int BK, int BN>
__global__ __launch_bounds__(256) void split_fixup_kernel(GemmParams p) {
    const int ntn = (p.N + BN - 1) / BN;
    const SplitPlan sp = split_plan<BK>(p, ntn, act_mtiles(p));
    if (sp.S < 2) return;
    constexpr int kSlabs = BM / 8;
    const int tid = threadIdx.x;
    const int rr = tid / (BN / 8), col = (tid % (BN / 8)) * 8;  // BN = 256: 8 rows x 32 lanes of 8 columns
    uint16_t* C = reinterpret_cast<uint16_t*>(p.c);
    for (int w = blockIdx.x; w < sp.R * kSlabs; w += gridDim.x) {
        const int j = w / kSlabs, slab = w % kSlabs;
        const int mt = sp.cut + j / ntn, nt = j % ntn;
        int e, row0 = 0, rows = 0;
        act_tile(p, mt, e, row0, rows);
        const int row = slab * 8 + rr;
        if (e < 0 || row >= rows || nt * BN + col >= p.N) continue;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        const float* src = p.part + (int64_t)j * sp.S * BM * BN + (int64_t)row * BN + col;
        // the loads of up to 8 parts in flight together (one round trip per
        // 8 parts), then added in part order
        for (int q0 = 0; q0 < sp.S; q0 += 8) {
            f32x4 a[8], b[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int q = min(q0 + u, sp.S - 1);  // clamped: the extra loads are not added
                a[u] = *reinterpret_cast<const f32x4*>(src + (int64_t)q * BM * BN);
                b[u] = *reinterpret_cast<const f32x4*>(src + (int64_t)q * BM * BN + 4);
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (q0 + u >= sp.S) break;
                acc[0] += a[u][0]; acc[1] += a[u][1]; acc[2] += a[u][2]; acc[3] += a[u][3];
                acc[4] += b[u][0]; acc[5] += b[u][1]; acc[6] += b[u][2]; acc[7] += b[u][3];
            }
        }
        *reinterpret_cast<uint4*>(C + (int64_t)(row0 + row) * p.ldc + nt * BN + col) = pack8(acc);
    }
}

}  // namespace

// Tile depth and ring per kind and tile width: split rings of K = 64 for the
// activation GEMMs on 256 columns; K = 32 rings otherwise (4 stages of 32 KiB
// at 256 columns, 3 of 24 KiB at 128 columns with two workgroups per CU).
// 128 x 128 tiles (two workgroups per CU, 64 KiB each, the size of the
// epilogue's staging anyway): 4 stages of K = 32, or with K64 2 stages of
// K = 64, whose 128-byte row segments the CU's load path takes at twice the
// rate of 64-byte ones (reference profile shape, K = 1280: up GEMM 25
// against 30 us; at K = 256 the deeper K = 32 ring is as fast or faster).
template <int KIND, int BN, int TBM = BM, bool K64 = false>
struct Ring {
    static constexpr bool split = split_ring<KIND, 64, BN, 2, TBM>();
    static constexpr bool k64 = K64 && TBM == 128;
    static constexpr int BK = split || k64 ? 64 : 32;
    static constexpr int NST = split ? 3 : k64 ? 2 : (BN == 256 || TBM == 128 ? 4 : 3);
};

// grid: the launch-order blocks of the tile map. Persistent kinds run
// min(grid, CUs rounded down to a multiple of 8) workgroups over them.
template <int KIND, bool DUAL, int BN, int NWM = 2, int TBM = BM, bool K64 = false>
hipError_t launch_kind(const GemmParams& p, unsigned grid, hipStream_t s) {
    using R = Ring<KIND, BN, TBM, K64>;
    GemmParams q = p;
    q.vblocks = (int)grid;
    unsigned g = grid;
    if constexpr (persistent_tiles<KIND, R::BK, BN, NWM, TBM>()) {
        const unsigned cus = (unsigned)(cu_count() / 8 * 8);
        if (cus >= 8 && g > cus) g = cus;
    }
    grouped_gemm_kernel<KIND, DUAL, R::BK, R::NST, BN, NWM, TBM><<<g, 128 * NWM, 0, s>>>(q);
    return hipGetLastError();
}

// Tile width per GEMM kind (BN 128 = two workgroups per CU). Measured in the
// c3 step: every GEMM runs fastest on 256-column tiles (UP, DOWN, DX and DACT
// on split rings; UP 1.26 against 1.29 ms with two 128-column workgroups per
// CU). DACT moved to 256 columns once its epilogue no longer evaluated
// silu'(U) itself (1.22 against 1.24 ms, and the weight-gradient GEMMs after
// it 0.02-0.04 ms faster); while it did, the co-resident second workgroup of
// the 128-column tiles covered that VALU work and won. The weight-gradient
// GEMMs run 256-column tiles in balanced 16-tile groups (4-6% faster than two
// 128-column workgroups).
// Small problems: a launch whose 256 x 256 tiles would leave most CUs idle
// runs 128 x 128 tiles (four times the tiles, two workgroups per CU). At
// the reference's profile shape (4096 slots, d = 1280, h = 0) the up GEMM
// took 30 us on 128 x 128 tiles against 29 us on 256 x 128 and 35 us on
// 256 x 256 (all with the XCD runs of launch_gemm_tile); at TMT's default
// width (2048 slots, d = 256) 9 against 12 and 16 us.
static int64_t tiles_256(GemmKind kind, const GemmParams& p) {
    const int64_t ntn = (p.N + 255) / 256;
    if (kind == GEMM_DW_DOWN || kind == GEMM_DW_UP) return (int64_t)p.E * ((p.M + BM - 1) / BM) * ntn;
    return ((int64_t)p.slots + BM - 1) / BM * ntn;  // lower bound (experts' partial tiles aside)
}

GemmTile gemm_tile(GemmKind kind, const GemmParams& p) {
    if (kind == GEMM_UP_FP4 || kind == GEMM_DOWN_FP4) return GemmTile{256, 256};
    if (2 * tiles_256(kind, p) < cu_count()) {
        const bool group_k = kind == GEMM_DW_DOWN || kind == GEMM_DW_UP;
        return GemmTile{128, 128, !group_k && p.K % 64 == 0 && p.K >= 512};
    }
    return GemmTile{256, 256};
}

hipError_t launch_gemm_tile(GemmKind kind, bool dual, const GemmParams& p, GemmTile tile, hipStream_t s) {
    const int bn = tile.n, bm = tile.m;
    if (p.N % 8 != 0 || p.N <= 0) return hipErrorInvalidValue;
    if (bn != 256 && bn != 128) return hipErrorInvalidValue;
    if (bm != 256 && !(bm == 128 && bn == 128)) return hipErrorInvalidValue;
    if (tile.k64 && (bm != 128 || p.K % 64 != 0 || kind == GEMM_DW_DOWN || kind == GEMM_DW_UP))
        return hipErrorInvalidValue;
    const bool group_k = kind == GEMM_DW_DOWN || kind == GEMM_DW_UP;
    const bool fp4 = kind == GEMM_UP_FP4 || kind == GEMM_DOWN_FP4;
    if (fp4 && (p.K % 64 != 0 || bn != 256 || bm != 256)) return hipErrorInvalidValue;
    const int64_t ntn = (p.N + bn - 1) / bn;
    const int64_t gn = ntn < 8 ? ntn : 8, gm = 32 / gn;
    const int64_t ngn = (ntn + gn - 1) / gn;
    int64_t groups;
    int64_t gsz = 32;  // tiles per group (weight-gradient GEMMs on 256 columns: 16)
    if (group_k) {
        if (p.M % 8 != 0 || p.M <= 0) return hipErrorInvalidValue;
        const int64_t ntm = (p.M + bm - 1) / bm;
        if (bn == 256) gsz = 16;
        const int64_t gmk = gsz / gn;
        groups = (int64_t)p.E * ((ntm + gmk - 1) / gmk) * ngn;
    } else {
        if (p.K % (bn == 256 && !fp4 ? 64 : 32) != 0) return hipErrorInvalidValue;
        // sum_e ceil(cnt_e / bm) <= ceil(slots / bm) + E - 1
        const int64_t mtiles = (int64_t)(p.slots + bm - 1) / bm + p.E;
        groups = ((mtiles + gm - 1) / gm) * ngn;
    }
    // whole rounds of 8 XCDs x 32 workgroups keep the block -> tile map a bijection
    int64_t grid = (groups * gsz + 255) / 256 * 256;
    GemmParams q = p;
    q.xcd_runs = 0;
    if (!group_k && !fp4) {
        // every tile resident at once (two workgroups per CU below 256 x 256):
        // 8 equal runs of tiles, one per XCD (at most 8 * ceil(tiles / 8) blocks)
        const int64_t mt_max = (int64_t)(p.slots + bm - 1) / bm + p.E;
        const int64_t tiles = mt_max * ntn;
        const int64_t slots_resident = (int64_t)cu_count() * (bn == 256 && bm == 256 ? 1 : 2);
        if (tiles <= slots_resident) {
            q.xcd_runs = 1;
            grid = (tiles + 7) / 8 * 8;
        }
    }
    // split-K tail (GEMM_DOWN / GEMM_DX on 256-column tiles): its parts are
    // the workgroups after the whole rounds, at most `resident` of them.
    const bool split = (kind == GEMM_DOWN || kind == GEMM_DX) && bn == 256 && bm == 256 && p.part != nullptr && !q.xcd_runs &&
                       p.resident > 0 && p.resident % 256 == 0;
    if (split) grid += p.resident;
    if (grid <= 0) return hipSuccess;
    if (grid > 0x7fffffff) return hipErrorInvalidValue;
    const unsigned g = (unsigned)grid;
#define TMT_BN(KIND_, DUAL_)                                      \
    (bn == 256     ? launch_kind<KIND_, DUAL_, 256>(q, g, s)      \
     : bm == 256   ? launch_kind<KIND_, DUAL_, 128>(q, g, s)      \
     : !tile.k64   ? launch_kind<KIND_, DUAL_, 128, 2, 128>(q, g, s) \
                   : launch_kind<KIND_, DUAL_, 128, 2, 128, true>(q, g, s))
    if (split) {
        // bn == 256 here, so launch_kind runs the 256-column kernel
        hipError_t err = kind == GEMM_DOWN ? launch_kind<GEMM_DOWN, false, 256>(q, g, s)
                                           : launch_kind<GEMM_DX, false, 256>(q, g, s);
        if (err != hipSuccess) return err;
        static_assert(Ring<GEMM_DOWN, 256>::BK == Ring<GEMM_DX, 256>::BK, "one split plan for DOWN and DX");
        // 4 workgroups per CU: the (tile, 8-row slab) items are short and latency-bound
        split_fixup_kernel<Ring<GEMM_DOWN, 256>::BK, 256><<<p.resident * 4, 256, 0, s>>>(q);
        return hipGetLastError();
    }
    switch (kind) {
        case GEMM_UP: return dual ? TMT_BN(GEMM_UP, true) : TMT_BN(GEMM_UP, false);
        case GEMM_DOWN: return TMT_BN(GEMM_DOWN, false);
        case GEMM_DACT: return TMT_BN(GEMM_DACT, false);
        case GEMM_DX: return TMT_BN(GEMM_DX, false);
        case GEMM_DW_DOWN: return TMT_BN(GEMM_DW_DOWN, false);
        case GEMM_DW_UP: return TMT_BN(GEMM_DW_UP, false);
        case GEMM_UP_FP4:
            return dual ? launch_kind<GEMM_UP_FP4, true, 256>(q, g, s) : launch_kind<GEMM_UP_FP4, false, 256>(q, g, s);
        case GEMM_DOWN_FP4: return launch_kind<GEMM_DOWN_FP4, false, 256>(q, g, s);
        default: return hipErrorInvalidValue;
    }
#undef TMT_BN
}

hipError_t launch_gemm(GemmKind kind, bool dual, const GemmParams& p, hipStream_t s) {
    return launch_gemm_tile(kind, dual, p, gemm_tile(kind, p), s);
}

}  // namespace tmt
