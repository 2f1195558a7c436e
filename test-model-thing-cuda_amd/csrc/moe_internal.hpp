// moe_internal.hpp -- shared declarations of the gfx950 MoE kernels.
//
// Kernel families (one .hip file each):
//   router.hip    router logits + softmax + top-k, block histograms, expert
//                 offset scan, stable token permutation
//   gemm.hip      grouped bf16 MFMA GEMMs over expert segments
//   skinny.hip    weight-streaming expert GEMMs for decode-sized batches
//   pointwise.hip combine, combine/router backward, router dW, dX scatter
//   norm.hip      LayerNorm forward / backward in front of the block
//   adamw.hip     multi-tensor AdamW with global-norm clipping
// The host orchestration lives in moe_api.cpp.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tmt {

constexpr int kMaxExperts = 64;
constexpr int kMaxTopK = 8;
constexpr int kThreads = 256;  // every kernel runs 4 waves of 64 ...
constexpr int kRouterWaves = 8;  // ... except the router: 8 waves share one staged Wr

// ---------------------------------------------------------------- router --
struct RouterParams {
    const uint16_t* X;     // [T][d] bf16
    const uint16_t* Wr;    // [E][d] bf16
    const float* bias;     // [E] or nullptr
    int T, d, E, K;
    int rows_per_block;    // multiple of kRouterWaves * (64 / EP)
    float* logits;         // [T][E]
    float* probs;          // [T][E]
    int32_t* idx;          // [T][K]
    float* gate;           // [T][K]
    float* lse;            // [T]
    int32_t* blkcnt;       // [nblk][E] picks per expert in each block
    float* blkstat;        // [nblk][E+1] sum of probs per expert, sum of lse^2
    // LayerNorm in front of the router (tmt_moe_forward_ln): X is then the
    // block input S, and the router also writes H, the LayerNorm output that
    // the expert GEMMs read, and the row statistics. ln_H == nullptr: X is the
    // router input itself.
    const float* ln_gamma;  // [d]
    const float* ln_beta;   // [d]
    uint16_t* ln_H;         // [T][d] bf16
    float* ln_mean;         // [T]
    float* ln_rstd;         // [T]
};
int router_ep(int E);  // padded expert count used by the router (power of 2)
// The router can run the LayerNorm of its rows itself (a wave's rows of S
// held in registers: rows per wave x 512-element chunks <= 16, d <= 2048).
bool router_ln_fits(int E, int d);
// Wr is staged in LDS by the router and the dX scatter when it fits in this
// many bytes; wider routers (E*d*2 larger) are read from global memory.
constexpr size_t kRouterWrLdsBytes = 65536;
inline bool router_wr_in_lds(int E, int d) { return (size_t)E * (size_t)d * 2 <= kRouterWrLdsBytes; }
int router_rows_per_wave(int E);
hipError_t launch_router(const RouterParams& p, int nblk, hipStream_t s);
// Large routed batches without the LayerNorm (router_mfma_fits): logits on
// the matrix cores, rows whose top-k ranking the MFMA rounding could change
// recomputed in the canonical order (picks bit-exact; logits within a few
// ulp elsewhere). rows_per_block must be kMfmaRouterRows.
constexpr int kMfmaRouterRows = 128;
bool router_mfma_fits(int T, int E, int K, int d);
hipError_t launch_router_mfma(const RouterParams& p, int nblk, hipStream_t s);

struct ScanParams {
    const int32_t* blkcnt;   // [nblk][E]
    const float* blkstat;    // [nblk][E+1]
    int nblk, T, E, K;
    int32_t* counts;         // [E]
    int32_t* offsets;        // [E+1]
    int32_t* blkbase;        // [nblk][E]
    int32_t* order;          // [E] experts by descending count (stable)
    float* stats;            // {aux, z} followed by E int32 counts
};
hipError_t launch_scan(const ScanParams& p, hipStream_t s);

struct PermuteParams {
    const int32_t* idx;      // [T][K]
    const int32_t* blkbase;  // [nblk][E]
    int T, E, K, rows_per_block;
    int32_t* perm;           // [T*K] slot -> token
    int32_t* slot_of;        // [T][K] (token, j) -> slot
};
hipError_t launch_permute(const PermuteParams& p, int nblk, hipStream_t s);
// scan + permute in one launch for nblk <= kFusedScanBlocks router blocks
// (blkbase is not written).
constexpr int kFusedScanBlocks = 64;
hipError_t launch_permute_scan(const PermuteParams& p, const ScanParams& sp, int nblk, hipStream_t s);

// T <= kSmallRouteTokens: router + scan + permute in one launch, one block
// per token row; with several rows the last block to finish (atomic
// *ticket, zero between calls and re-armed by that block) completes the
// dispatch. Uses sp.counts/offsets/order/stats and pp.perm/slot_of; no
// block tables. With ticket == nullptr and T > 1 the blocks only write their
// rows' picks (idx, gate, logits, probs, lse): the decode GEMM_UP completes
// the dispatch (GemmParams::self_dispatch).
constexpr int kSmallRouteTokens = 64;
hipError_t launch_route_small(const RouterParams& p, const ScanParams& sp, const PermuteParams& pp,
                              int* ticket, hipStream_t s);

// E == 1: identity dispatch, gates of 1, offsets {0, T}.
hipError_t launch_dense_dispatch(int T, int32_t* perm, int32_t* slot_of,
                                 float* gate, int32_t* counts, int32_t* offsets,
                                 int32_t* order, float* stats, hipStream_t s);

// ------------------------------------------------------------------ gemm --
enum GemmKind {
    GEMM_UP = 0,       // C = gather(X) W_up^T        (+ SiLU copy when dual)
    GEMM_DOWN = 1,     // C = A W_down^T
    GEMM_DACT = 2,     // C = (dO W_down) * silu'(U)
    GEMM_DX = 3,       // C = dU W_up
    GEMM_DW_DOWN = 4,  // dW_down[e] = dO^T A            (reduction over slots)
    GEMM_DW_UP = 5,    // dW_up[e]   = dU^T Xg           (reduction over slots)
    GEMM_UP_FP4 = 6,   // GEMM_UP with MXFP4 weights dequantised to bf16 in registers
    GEMM_DOWN_FP4 = 7  // GEMM_DOWN with MXFP4 weights
};

struct GemmParams {
    const int32_t* offsets;  // [E+1] expert segment starts (slot space)
    const int32_t* order;    // [E] processing order for weight-gradient GEMMs
    const int32_t* perm;     // [TK] slot -> token (gather table)
    const int32_t* idx;      // decode UP: [T][topk] expert picks (nullptr: slot == token)
    int topk;
    int E;
    int M;                   // weight-gradient GEMMs: rows of C
    int N;                   // columns of C
    int K;                   // activation GEMMs: reduction length
    int slots;               // activation GEMMs: T*K routed rows (bounds the row tiles)
    const uint16_t* a; int64_t lda;   // activation operand
    const uint16_t* b; int64_t ldb;   // second activation operand (dW GEMMs)
    void* c; int64_t ldc;             // output (activation GEMMs)
    uint16_t* c2;                     // GEMM_UP with hidden > 0: SiLU(U) (c then gets silu'(U))
    const uint16_t* u;                // GEMM_DACT: silu'(U) as the up GEMM wrote it
    const uint16_t* w[kMaxExperts];   // per-expert weights (activation GEMMs)
    float* dw[kMaxExperts];           // per-expert fp32 outputs (dW GEMMs)
    const uint8_t* wq[kMaxExperts];   // MXFP4 weights: packed e2m1 [N][K/2] (low nibble = even k)
    const uint8_t* wsc[kMaxExperts];  // MXFP4 scales: e8m0 [K/32][N]
    // GEMM_DOWN / GEMM_DX: split-K of the last round's tiles. part holds
    // resident * BM * BN fp32 partial tiles (nullptr: no split); resident is
    // the number of workgroups the GPU runs at once (one per CU).
    float* part;
    int resident;
    // Decode GEMM_DOWN (skinny kernels): [2][slots][N] fp32 buffer for a
    // split of K into two halves (nullptr: no split).
    float* dpart;
    // Decode batches with self_dispatch (skinny stream kernels): the router
    // wrote only the picks; workgroup (e, s) takes expert e's rows straight
    // from the [T][topk] pick table in idx (the grid is indexed by expert).
    int self_dispatch;
    // Set by the launcher: launch-order blocks of the tile map (persistent
    // grouped GEMMs loop over them).
    int vblocks;
    // Set by the launcher for activation GEMMs whose tiles all run at once:
    // the (M tile, N tile) list is cut into 8 equal runs, one per XCD.
    int xcd_runs;
};
hipError_t launch_gemm(GemmKind kind, bool dual, const GemmParams& p, hipStream_t s);
// Rows of an activation-GEMM tile, and the fp32 partial buffer the split-K
// tail needs (floats) for `resident` workgroups.
constexpr int kGemmTileRows = 256;
inline size_t gemm_split_floats(int resident) { return (size_t)resident * kGemmTileRows * 256; }
int cu_count();  // compute units of the current device (cached per device)
// Same with an explicit tile shape: 256 x 256 (one workgroup per CU),
// 256 x 128 or 128 x 128 (two workgroups per CU; bf16 kinds only).
struct GemmTile {
    int m, n;
    bool k64 = false;  // 128 x 128 tiles: 2 stages of K = 64 instead of 4 of K = 32
};
GemmTile gemm_tile(GemmKind kind, const GemmParams& p);  // the shape launch_gemm picks
hipError_t launch_gemm_tile(GemmKind kind, bool dual, const GemmParams& p, GemmTile tile, hipStream_t s);

// Decode-sized forward GEMMs (GEMM_UP / GEMM_DOWN, bf16 weights) for
// T <= kSkinnyMaxTokens tokens: every expert then owns at most T rows.
constexpr int kSkinnyMaxTokens = 64;
// With p.dpart set, GEMM_DOWN may split K in halves (*halves = true): the
// outputs are then the two fp32 partial rows in p.dpart, not bf16 rows in
// p.c, and the combine adds them (CombineParams::part).
hipError_t launch_skinny_gemm(GemmKind kind, bool dual, const GemmParams& p, int T, hipStream_t s,
                              bool* halves = nullptr);
// One-token decode: GEMM_DOWN of the token's K experts and the combine in
// one launch. Workgroup b owns output columns 4b .. 4b+3 for all K picks, so
// the combine needs no other workgroup's results. Needs K <= 8, h % 256 == 0
// with 4 <= h / 256 <= 16, and d % 4 == 0.
struct Down1Params {
    const uint16_t* w[kMaxExperts];  // W_down[e] [d][h]
    const uint16_t* a;               // SiLU(U) rows in slot order [K][h]
    const int32_t* idx;              // [K] the token's experts
    const float* gate;               // [K]
    const int32_t* slot_of;          // [K]
    uint16_t* O;                     // [K][d] expert outputs in slot order (kept for the backward)
    uint16_t* Y;                     // [1][d]
    float beta;
    int d, h, K;
};
bool decode1_down_combine_fits(int d, int h, int K);
hipError_t launch_decode1_down_combine(const Down1Params& p, hipStream_t s);
// One-token decode: GEMM_UP routes its token itself, with the arithmetic of
// route_small_kernel's single-token path (every workgroup computes the picks
// it needs; workgroup 0 also writes the router outputs and the dispatch
// tables), so no router launch precedes it. Needs E > 1 and a chunk
// kernel reduction shape (d % 256 == 0 with 4 <= d / 256 <= 16, or
// d % 64 == 0 with d / 64 <= 16).
struct Route1 {
    RouterParams rp;
    ScanParams sp;
    PermuteParams pp;
};
bool skinny_up_route1_fits(int d, int E);
hipError_t launch_skinny_up_route1(bool dual, const GemmParams& p, const Route1& r, hipStream_t s);

// Whether a decode forward of these shapes runs every expert GEMM on the
// skinny stream kernel (the kernel that supports self_dispatch): GEMM_UP
// with hn output columns and, with h > 0, GEMM_DOWN (K = h, N = d).
bool skinny_self_dispatch(int T, int E, int K, int d, int h, int hn);

// ------------------------------------------------------------- gemm_mx ----
// MXFP4 weights times activations held as two MXFP6 terms, on the scaled
// MFMA (layouts in gemm_mx.hip). Activation tensors ("MX6x2") are held in
// K planes of 64: codes [K/64][srows][96] bytes, scales [K/64][srows][4]
// bytes, srows >= rows + kMxScalePadRows.
constexpr int kMxScalePadRows = 256;
inline size_t mx_codes_bytes(int64_t rows, int64_t K) {
    return (size_t)(K / 64) * (size_t)(rows + kMxScalePadRows) * 96;
}
inline size_t mx_scales_bytes(int64_t rows, int64_t K) {
    return (size_t)(K / 64) * (size_t)(rows + kMxScalePadRows) * 4;
}
struct MxQuantParams {
    const uint16_t* X;       // bf16 rows (tokens)
    int64_t ldx;
    const int32_t* slot_of;  // [rows][copies]: the slots row r is written to (nullptr: slot r)
    int copies;              // slots per row (1 when slot_of is nullptr)
    int rows, K;
    uint8_t* codes;          // [K/64][srows][96]
    uint8_t* scales;         // [K/64][srows][4]
    int64_t srows;
};
hipError_t launch_mx_quant_rows(const MxQuantParams& p, hipStream_t s);
// MXFP4 weight codes [N][K/2] (the caller's layout) to K planes of 64:
// [K/64][N][32] bytes per expert, for two matrix sets (w = 0, 1) at once.
struct MxPlanesParams {
    const uint8_t* src[2][kMaxExperts];
    uint8_t* dst[2];  // expert e at dst[w] + e * N[w] * K[w] / 2
    int N[2], K[2];   // N[w] == 0: set w is empty
    int E;
};
hipError_t launch_mx_weight_planes(const MxPlanesParams& p, hipStream_t s);
struct MxGemmParams {
    const int32_t* offsets;  // [E+1] expert segments (slot space)
    int E;
    int N, K, slots;         // output columns, reduction length, routed rows
    const uint8_t* a_codes;  // activations, MX6x2 planes in slot order (srows = a_srows)
    const uint8_t* a_scales;
    int64_t a_srows;
    const uint8_t* wq[kMaxExperts];   // e2m1 codes in K planes [K/64][N][32] per expert
    const uint8_t* wsc[kMaxExperts];  // e8m0 scales [K/32][N] per expert
    uint16_t* c;             // bf16 output [slots][ldc] (quant_out == false)
    int64_t ldc;
    uint8_t* q_codes;        // SiLU(output) as MX6x2 planes, slot order (quant_out == true)
    uint8_t* q_scales;
    int64_t q_srows;
};
hipError_t launch_mx_gemm(bool quant_out, const MxGemmParams& p, hipStream_t s);

// ------------------------------------------------------------- pointwise --
// Dispatch tables of a decode batch written from the pick table on the GPU
// (dispatch.hpp): the outputs of the router's dispatch, and the router
// outputs the aux / z statistics are summed from.
struct DispatchTables {
    int T, E, K;
    const float* probs;  // [T][E]
    const float* lse;    // [T]
    int32_t* offsets;    // [E+1]
    int32_t* counts;     // [E]
    int32_t* order;      // [E] experts by descending count (ties: lower index first)
    int32_t* perm;       // [T*K] slot -> token
    int32_t* slot_of;    // [T][K]
    float* stats;        // aux, z, then the counts as int32
};

struct CombineParams {
    const uint16_t* O;       // [TK][d] expert outputs (hidden > 0) or U (hidden == 0)
    const int32_t* slot_of;  // [T][K]
    const float* gate;       // [T][K]
    uint16_t* Y;             // [T][d]
    float beta;
    int T, d, K;
    int silu;                // 1: apply SiLU to O (hidden == 0)
    // Decode GEMM_DOWN split in K halves: O[slot] = bf16(part[0][slot] +
    // part[1][slot]) is formed here and also stored to O_out (nullptr part:
    // O is read as is).
    const float* part;       // [2][slots][d]
    uint16_t* O_out;         // [slots][d]
    int slots;
    // Decode batches with self_dispatch (T <= kSkinnyMaxTokens): each row
    // finds its picks' slots from the [T][K] pick table in idx instead of
    // slot_of, and one extra workgroup writes the dispatch tables.
    int self_dispatch;
    const int32_t* idx;
    DispatchTables tables;
};
hipError_t launch_combine(const CombineParams& p, hipStream_t s);

struct CombineBwdParams {
    const uint16_t* dY;      // [T][d]
    const uint16_t* O;       // [TK][d] (hidden > 0) or U (hidden == 0)
    const int32_t* slot_of;  // [T][K]
    const int32_t* idx;      // [T][K]
    const float* gate;       // [T][K]
    const float* probs;      // [T][E]
    const float* lse;        // [T]
    const int32_t* counts;   // [E]
    int T, d, E, K;
    int silu;                // 1: hidden == 0 (SiLU applied in combine)
    float aux_coef, z_coef;
    uint16_t* dO;            // [TK][d] gradient at the expert output
    float* dlogits;          // [T][E] (E > 1)
    const uint16_t* X;       // [T][d] layer input
    uint16_t* Xg;            // [TK][d] X gathered to slot order (dW_up operand)
};
hipError_t launch_combine_bwd(const CombineBwdParams& p, hipStream_t s);

struct RouterDwParams {
    const float* dlogits;    // [T][E]
    const uint16_t* X;       // [T][d]
    int T, d, E;
    int nchunks;
    float* partial;          // [nchunks][E][d]
    float* dWr;              // [E][d]
};
int router_dw_chunks(int T, int E, int d);
int router_dw_chunks_max(int max_tokens, int E, int d);
// reduce = false: pass 1 only; the scatter's launch then runs pass 2
// (ScatterParams::dw).
hipError_t launch_router_dw(const RouterDwParams& p, hipStream_t s, bool reduce = true);

struct ScatterParams {
    const uint16_t* dXg;     // [TK][d]
    const int32_t* slot_of;  // [T][K]
    const float* dlogits;    // [T][E] or nullptr
    const uint16_t* Wr;      // [E][d]
    int T, d, E, K;
    uint16_t* dX;            // [T][d] (unused when the LayerNorm backward is fused)
    // LayerNorm backward fused into the scatter (ln_S != nullptr, d <= kLnFusedMaxD):
    // the bf16-rounded dX row is the gradient at the LayerNorm output.
    const uint16_t* ln_S;    // [T][d] LayerNorm input
    const float* ln_gamma;   // [d]
    const float* ln_mean;    // [T]
    const float* ln_rstd;    // [T]
    uint16_t* ln_dS;         // [T][d]
    float* ln_partial;       // [scatter_blocks(T)][2][d] per-block dgamma / dbeta sums
    // Pass 2 of the router weight gradient (the per-output sum over pass 1's
    // chunks) run by extra workgroups of the same launch (dw.partial !=
    // nullptr; only without the LayerNorm): the two are independent, and
    // one launch fewer shortens a small backward.
    RouterDwParams dw;
};
constexpr int kLnFusedMaxD = 2048;
constexpr int kScatterRows = 64;  // rows per scatter workgroup (router or LayerNorm variants)
int scatter_blocks(int T);
hipError_t launch_scatter(const ScatterParams& p, hipStream_t s);

// p[0, n) = 0 with a kernel (no memset node, so the call can be captured).
hipError_t launch_zero_f32(float* p, int64_t n, hipStream_t s);
// out = bf16(in), round to nearest even.
hipError_t launch_f32_to_bf16(const float* in, uint16_t* out, int64_t n, hipStream_t s);
// dst + e * rows * cols = src[e]^T ([rows][cols] bf16, row stride ld_src ->
// [cols][rows]); rows and cols multiples of 64.
struct TransposeParams {
    const uint16_t* src[kMaxExperts];
    int64_t ld_src;
    int rows, cols;
    uint16_t* dst;
};
hipError_t launch_transpose_bf16(const TransposeParams& p, int nmat, hipStream_t s);

// ------------------------------------------------------------------ norm --
struct LayerNormParams {
    const uint16_t* S;       // [T][lds] bf16 LayerNorm input (d columns used)
    const float* gamma;      // [d]
    const float* beta;       // [d] (forward)
    int T, d;                // rows, row width (the statistics divide by d)
    int lds, ldh;            // row strides of S / dS and of H / dH (>= d); H's
                             // columns [d, ldh) are written as zeros
    uint16_t* H;             // [T][ldh] bf16 output (forward)
    float* mean;             // [T] (written by forward, read by backward)
    float* rstd;             // [T]
    const uint16_t* dH;      // [T][ldh] bf16 gradient at H (backward)
    uint16_t* dS;            // [T][lds] bf16 (backward)
    float* partial;          // [ln_chunks(T)][2][ln_width4(d)] dgamma / dbeta chunk sums
    float* partial2;         // [colsum_groups(ln_chunks(T))][2][ln_width4(d)] (level-1 sums)
    float* dgamma;           // [d]
    float* dbeta;            // [d]
};
int ln_chunks(int T);
// Row stride of the dgamma / dbeta partials: d rounded up to a multiple of 4.
__host__ __device__ inline int ln_width4(int d) { return (d + 3) & ~3; }
hipError_t launch_ln_fwd(const LayerNormParams& p, hipStream_t s);
hipError_t launch_ln_bwd(const LayerNormParams& p, hipStream_t s);
// Fixed-order column sums of in [nrows][ncols] (ncols % 4 == 0): columns
// [0, split) to out_lo, [split, ncols) to out_hi, each of which receives its
// first `width` columns (width <= split, ncols - split); scratch holds
// [colsum_groups(nrows)][ncols] level-1 sums.
int colsum_groups(int nrows);
hipError_t launch_colsum(const float* in, int nrows, int ncols, float* scratch, int split, int width,
                         float* out_lo, float* out_hi, hipStream_t s);

// Zero-padded copies between a caller's matrices and the internal ones of a
// handle whose width is not a multiple of 64: dst[r][c] = src[r][c] for
// r < rows_s and c < cols_s, else 0, over rows_d x cols_d (one launch copies
// up to kMaxExperts matrices of one shape; blockIdx.y picks the matrix).
struct PadParams {
    const void* src[kMaxExperts];
    void* dst[kMaxExperts];
    int64_t rows_s, cols_s, ld_s;
    int64_t rows_d, cols_d, ld_d;
};
hipError_t launch_pad_copy(const PadParams& p, int nmat, int elem_bytes, hipStream_t s);

// ----------------------------------------------------------------- adamw --
constexpr int kAdamChunk = 8192;      // elements per chunk (one workgroup)
constexpr int kAdamwInNorm = 1;       // flags bit 0: gradient counts in the clipping norm
constexpr int kAdamwUpdate = 2;       // flags bit 1: parameter is updated
struct AdamwChunk {
    float* master;                    // chunk start in each tensor (16-byte aligned)
    float* m;
    float* v;
    float* grad;
    uint16_t* work;                   // bf16 working copy or nullptr
    int32_t len;                      // elements, <= kAdamChunk
    int32_t flags;
};
struct AdamwParams {
    const AdamwChunk* chunks;         // [nchunks]
    int nchunks;
    double* partial;                  // [nchunks] per-chunk sums of grad^2
    double* sumsq;                    // global sum of grad^2
};
struct AdamwHyper {
    float clip, lr, b1, b2, eps, wd, bc1, bc2;
};
hipError_t launch_adamw_sumsq(const AdamwParams& p, hipStream_t s);
hipError_t launch_adamw_update(const AdamwParams& p, const AdamwHyper& h, hipStream_t s);
hipError_t launch_adamw_zero(const AdamwParams& p, hipStream_t s);

}  // namespace tmt
