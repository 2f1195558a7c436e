// skinny.hip -- grouped expert GEMMs for decode-sized batches (gfx950).
//
// With T <= 64 tokens every expert owns at most T rows, so the expert GEMMs
// are weight-streaming problems (the reference runs them as padded 128-row
// cuBLAS calls, tmt-cuda/src/moe.cu:414-436, tmt-cuda/src/generate.h:19-44).
// The 256 x 256 tiles of gemm.hip would leave most CUs idle and read each
// weight tile through a deep LDS pipeline for one useful row. Here a
// workgroup owns one or two tiles of 16 output columns of one expert and all
// of its rows:
//   * the waves split the reduction (K) into contiguous chunks;
//   * each lane streams weight rows (output columns) straight from HBM into
//     registers, and the matching activation row of each 16-row block (rows
//     past the expert's count are zero and not loaded);
//   * v_mfma_f32_16x16x32_bf16 multiplies them. A and B use the same
//     lane/k assignment, which is a permutation of the reduction, so the
//     product is the plain dot product;
//   * the wave partials are summed in LDS in a fixed order and written with
//     the same epilogue semantics as gemm.hip (U, SiLU(U) from the fp32 sum).
// skinny_chunk_kernel is the main path; skinny_gemm_kernel covers reduction
// lengths that do not split into one chunk per wave.
// Experts are visited in descending-count order (the scan's LPT order), so
// the grid only spans min(E, T*K) expert ranks.
//
// Decode steps are latency-bound, so a workgroup's first memory round trip
// fetches everything its loads depend on: the rank's expert, the whole
// offset table and the per-expert weight pointers (lane e holds expert e's
// entries, the rank's expert is then picked from registers) and, for UP,
// the [T][K] pick table, from which each wave finds the tokens of its
// expert's rows itself instead of reading the permutation (a second round
// trip before the activation loads).
#include "device_util.hpp"
#include "dispatch.hpp"
#include "route_row.hpp"
#include "moe_internal.hpp"

namespace tmt {
namespace {

__device__ __forceinline__ uint4 ld16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }

__device__ __forceinline__ f32x4 mfma16(const uint4& w, const uint4& a, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, w),
                                                   __builtin_bit_cast(bf16x8, a), c, 0, 0, 0);
}

// Weight streams go through a buffer resource: a pointer picked from
// registers is no longer known to be global memory, so plain loads through
// it would become flat loads, which also count on the LDS/scalar counter and
// so hold up every later LDS or scalar wait; buffer loads count on the
// vector-memory counter only. Word 3 is the gfx9 raw-buffer format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t weight_rsrc(const uint16_t* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), 0, bytes, 0x00020000);
}
__device__ __forceinline__ uint4 ld16_buf(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// One output element: the up GEMM with hidden > 0 (DUAL) writes silu'(U) to C
// and SiLU(U) to c2 (U itself is not kept: the backward only needs silu'(U));
// otherwise C = v.
template <bool DUAL>
__device__ __forceinline__ void store_up(uint16_t* C, uint16_t* c2, int64_t off, float v) {
    if constexpr (DUAL) {
        float a, da;
        silu_dsilu(v, a, da);
        C[off] = f2bf(da);
        c2[off] = f2bf(a);
    } else {
        C[off] = f2bf(v);
    }
}

// Kernel arguments are brought into registers before the first data load:
// a scalar argument load that the compiler sinks below the table loads
// would add a round trip to the workgroup's critical path.
__device__ __forceinline__ void in_sgpr(int v) { asm volatile("" ::"s"(v)); }
__device__ __forceinline__ void in_sgpr(int64_t v) { asm volatile("" ::"s"(v)); }
__device__ __forceinline__ void in_sgpr(const void* v) { asm volatile("" ::"s"(v)); }
template <class... T>
__device__ __forceinline__ void args_in_sgprs(const T&... v) {
    (in_sgpr(v), ...);
}

// The expert of one rank: its first slot, row count and weights.
struct SkinnyExpert {
    int e, row0, rows;
    const uint16_t* w;
};

// All four tables are read with vector loads: a scalar load of order[rank]
// would share its wait counter with the kernel-argument loads that the
// compiler places between the table loads, and so serialise them.
__device__ __forceinline__ SkinnyExpert skinny_expert(const GemmParams& p, int rank, int lane) {
    const bool in = lane < p.E;
    const int ov = in ? p.order[lane] : 0;
    const int o0 = in ? p.offsets[lane] : 0;
    const int o1 = in ? p.offsets[lane + 1] : 0;
    const uint64_t wl = in ? reinterpret_cast<uint64_t>(p.w[lane]) : 0;
    SkinnyExpert x;
    x.e = __builtin_amdgcn_readlane(ov, rank);
    x.row0 = __builtin_amdgcn_readlane(o0, x.e);
    x.rows = __builtin_amdgcn_readlane(o1, x.e) - x.row0;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)wl, x.e);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(wl >> 32), x.e);
    x.w = reinterpret_cast<const uint16_t*>(((uint64_t)hi << 32) | lo);
    return x;
}

// The [T][K] pick table (dispatch.hpp), entries q * 64 + lane.
__device__ __forceinline__ void load_picks(const GemmParams& p, int lane, int (&ent)[kPickGroups]) {
    load_pick_table(p.idx, p.slots, lane, ent);
}

// tok[m] = token of row m of expert e, for the first 16 * RB rows. The
// dispatch is stable (an expert's slots follow ascending token order) and a
// token picks an expert at most once, so row m is the m-th pick of e in
// table order. The list is the wave's own: LDS accesses of one wave complete
// in order, so no barrier is needed before the wave reads it back.
__device__ __forceinline__ void expert_tokens(const int (&ent)[kPickGroups], int slots, int K, int e,
                                              int lane, int maxrows, int* tok) {
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int base = 0;
#pragma unroll
    for (int q = 0; q < kPickGroups; ++q) {
        if (q * 64 >= slots) break;  // uniform
        const bool hit = ent[q] == e;
        const uint64_t mk = __ballot(hit);
        const int r = base + __popcll(mk & lt);
        if (hit && r < maxrows) tok[r] = (q * 64 + lane) / K;
        base += __popcll(mk);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// self_dispatch: expert e's first slot and row count from the pick table.
__device__ __forceinline__ SkinnyExpert self_expert(const GemmParams& p, int e, const int (&ent)[kPickGroups]) {
    SkinnyExpert x;
    x.e = e;
    expert_span(ent, p.slots, e, x.row0, x.rows);
    x.w = p.w[e];
    return x;
}

template <int KIND, bool DUAL, int RB>
__global__ __launch_bounds__(kThreads) void skinny_gemm_kernel(GemmParams p, int nexp) {
    static_assert(KIND == GEMM_UP || KIND == GEMM_DOWN, "forward GEMMs only");
    constexpr bool kGather = KIND == GEMM_UP;
    __shared__ f32x4 red[4][RB][64];
    __shared__ int s_tok[4][16 * RB];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rank = (int)blockIdx.x % nexp, tile = (int)blockIdx.x / nexp;
    int ent[kPickGroups];
    if constexpr (kGather) load_picks(p, lane, ent);
    const SkinnyExpert x = skinny_expert(p, rank, lane);
    const int row0 = x.row0;
    const int rows = min(x.rows, 16 * RB);
    if (rows <= 0) return;
    const int n0 = tile * 16;
    const int g = lane >> 4, li = lane & 15;
    if constexpr (kGather) {
        if (p.idx != nullptr) expert_tokens(ent, p.slots, p.topk, x.e, lane, 16 * RB, s_tok[wave]);
    }

    // This lane's weight row (output column n0 + li) and activation rows.
    const uint16_t* wrow = p.w[x.e] + (int64_t)(n0 + li) * p.ldb;  // kernarg pointer: global loads
    const uint16_t* arow[RB];
    bool aok[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int m = rb * 16 + li;
        aok[rb] = m < rows;
        const int mm = aok[rb] ? m : 0;
        const int src = (kGather && p.idx != nullptr) ? s_tok[wave][mm] : row0 + mm;
        arow[rb] = p.a + (int64_t)src * p.lda;
    }

    // The wave's share of the reduction, in units of 64 elements.
    const int units = p.K >> 6;
    const int u0 = wave * units / 4, u1 = (wave + 1) * units / 4;
    f32x4 acc[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint4 zero = make_uint4(0, 0, 0, 0);

    // Chunks of 4 units (256 elements): lane group g covers 64 contiguous
    // elements, i.e. 8 x 16-byte loads of its weight row. The next chunk's
    // weights are requested before the current chunk's MFMAs.
    int u = u0;
    if (u + 4 <= u1) {
        uint4 wv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) wv[i] = ld16(wrow + u * 64 + g * 64 + 8 * i);
        for (; u + 4 <= u1; u += 4) {
            const int kb = u * 64 + g * 64;
            uint4 wn[8];
            const bool more = u + 8 <= u1;
#pragma unroll
            for (int i = 0; i < 8; ++i) wn[i] = more ? ld16(wrow + kb + 256 + 8 * i) : zero;
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                uint4 av[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) av[i] = aok[rb] ? ld16(arow[rb] + kb + 8 * i) : zero;
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[rb] = mfma16(wv[i], av[i], acc[rb]);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) wv[i] = wn[i];
        }
    }
    // Remaining single units: lane group g covers 16 elements.
    for (; u < u1; ++u) {
        const int kb = u * 64 + g * 16;
        const uint4 w0 = ld16(wrow + kb), w1 = ld16(wrow + kb + 8);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const uint4 a0 = aok[rb] ? ld16(arow[rb] + kb) : zero;
            const uint4 a1 = aok[rb] ? ld16(arow[rb] + kb + 8) : zero;
            acc[rb] = mfma16(w0, a0, acc[rb]);
            acc[rb] = mfma16(w1, a1, acc[rb]);
        }
    }

    // acc[rb][r] = C[row rb*16 + li][column n0 + 4g + r] (16x16 MFMA layout:
    // first-operand index 4*(lane/16) + r, second-operand index lane % 16).
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) red[wave][rb][lane] = acc[rb];
    __syncthreads();

    // Thread t -> row m = t / 16, column n = t % 16 of each row block; the four
    // wave partials are added in wave order.
    const int m = tid >> 4, n = tid & 15;
    const int src_lane = (n >> 2) * 16 + m, r = n & 3;
    uint16_t* C = reinterpret_cast<uint16_t*>(p.c);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int row = rb * 16 + m;
        if (row >= rows) continue;
        float v = red[0][rb][src_lane][r];
        v += red[1][rb][src_lane][r];
        v += red[2][rb][src_lane][r];
        v += red[3][rb][src_lane][r];
        const int64_t off = (int64_t)(row0 + row) * p.ldc + n0 + n;
        store_up<DUAL>(C, p.c2, off, v);
    }
}

// Output column tiles of 16 per workgroup in the chunk kernel (CT): with
// two, both tiles' weight loads are in flight together and each activation
// chunk is loaded once for both (measured with d = 1024, h = 4096, E = 16,
// top-4: T = 64 UP 40.6 -> 30.6 us, DOWN 42.0 -> 31.1 us, T = 8 about 10%
// faster; four tiles are slower again). Below kSkinnyTwoTileTokens tokens
// the step is latency-bound and the larger grid of one tile wins (T = 1:
// 29.6 us per step with one tile, 34.0 with two).
constexpr int kSkinnyTwoTileTokens = 4;
// From this many tokens the persistent kernel (skinny_stream_kernel) runs
// where it applies.
constexpr int kSkinnyStreamTokens = 4;

// Variant for reduction lengths K = NW * 32J (J = 8: K a multiple of 256
// up to 4096; J = 2: a multiple of 64 up to 1024): the workgroup has NW
// waves and wave w owns one K-chunk, [32Jw, 32J(w+1)); lane group g holds
// k = 32Jw + 32i + 8g .. +7 for MFMA i, so the four lane groups of one load
// instruction read 64 contiguous bytes of each of the 16 rows (16 cache
// lines per instruction instead of 64: the address unit, not HBM, bounded
// the first layout). Every weight load of the tile is
// issued at once (J per lane), then each 16-row block of the expert loads
// its activation chunk and multiplies; blocks past the expert's count are
// skipped as a whole (uniform branch). No load sits under a divergent
// branch, so the compiler's wait counts stay exact.
// EP1 > 0 (GEMM_UP of one token, launch_skinny_up_route1): the workgroup
// routes the token itself -- logits over its waves, softmax and top-k on EP1
// lanes of wave 0 -- and takes the rank-th picked expert in ascending index
// (the slot order); workgroup 0 also writes the router outputs and tables.
template <int KIND, bool DUAL, int J, int RB, int CT, int EP1 = 0>
__global__ __launch_bounds__(1024) void skinny_chunk_kernel(GemmParams p, int nexp, Route1 r1) {
    static_assert(KIND == GEMM_UP || KIND == GEMM_DOWN, "forward GEMMs only");
    static_assert(EP1 == 0 || (KIND == GEMM_UP && RB == 1), "self-routing: the one-token GEMM_UP");
    constexpr bool kGather = KIND == GEMM_UP;
    extern __shared__ f32x4 red[];  // [RB][CT][nw][64] wave partials
    __shared__ int s_tok[16][16 * RB];

    const int nw = (int)blockDim.x >> 6;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rank = (int)blockIdx.x % nexp, tile0 = ((int)blockIdx.x / nexp) * CT;
    args_in_sgprs(p.order, p.offsets, p.idx, p.a, p.c, p.c2, p.E, p.slots, p.topk, p.lda, p.ldb, p.ldc);
    int ent[kPickGroups];
    SkinnyExpert x;
    if constexpr (EP1 > 0) {
        __shared__ float s_logit1[kMaxExperts];
        __shared__ int s_e1;
        token_logits(r1.rp, 0, s_logit1, wave, nw, lane);
        __syncthreads();
        if (wave == 0) {
            const int e = lane % EP1;
            const bool ev = lane < EP1 && e < r1.rp.E;
            const float logit = ev ? s_logit1[e] : 0.0f;
            const RowPick pk = softmax_topk<EP1>(logit, ev, e, r1.rp.K);
            if (blockIdx.x == 0) one_token_dispatch<EP1>(r1.rp, r1.sp, r1.pp, logit, ev, pk, lane);
            uint64_t selm = __ballot(ev && pk.sel);
            for (int i = 0; i < rank; ++i) selm &= selm - 1;  // drop the rank lowest picks
            if (lane == 0) s_e1 = (int)__builtin_ctzll(selm);
        }
        __syncthreads();
        x.e = __builtin_amdgcn_readfirstlane(s_e1);
        x.row0 = rank;  // a single token's slots follow ascending expert index
        x.rows = 1;
        x.w = p.w[x.e];
    } else {
        if constexpr (kGather) load_picks(p, lane, ent);
        x = skinny_expert(p, rank, lane);
    }
    const int row0 = x.row0;
    const int rows = min(x.rows, 16 * RB);
    if (rows <= 0) return;
    const int nrb = (rows + 15) >> 4;
    const int g = lane >> 4, li = lane & 15;
    const int kw = wave * (32 * J) + g * 8;

    // The workgroup's CT * 16 weight rows (K <= 4096 on this path: at most
    // 256 KiB, so 32-bit offsets).
    const __amdgpu_buffer_rsrc_t wr = weight_rsrc(x.w + (int64_t)tile0 * 16 * p.ldb, CT * 16 * (int)p.ldb * 2);
    uint4 wv[CT][J];
#pragma unroll
    for (int c = 0; c < CT; ++c) {
        const int off = ((c * 16 + li) * (int)p.ldb + kw) * 2;
#pragma unroll
        for (int i = 0; i < J; ++i) wv[c][i] = ld16_buf(wr, off + 64 * i);
    }
    const bool by_pick = kGather && EP1 == 0 && p.idx != nullptr;
    if (by_pick) expert_tokens(ent, p.slots, p.topk, x.e, lane, 16 * RB, s_tok[wave]);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        if (rb >= nrb) break;  // uniform
        const int m = rb * 16 + li;
        const bool ok = m < rows;
        const int mm = ok ? m : 0;
        const int srow = EP1 > 0 ? 0 : (by_pick ? s_tok[wave][mm] : row0 + mm);
        const uint16_t* ar = p.a + (int64_t)srow * p.lda + kw;
        uint4 av[J];
#pragma unroll
        for (int i = 0; i < J; ++i) av[i] = ld16(ar + 32 * i);
        if (!ok) {
#pragma unroll
            for (int i = 0; i < J; ++i) av[i] = make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < CT; ++c) {
            f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < J; ++i) acc = mfma16(wv[c][i], av[i], acc);
            red[((rb * CT + c) * nw + wave) * 64 + lane] = acc;
        }
    }
    __syncthreads();

    // Output (m, n) of a row block and column tile = lane (n/4)*16 + m,
    // element n%4; the wave partials are added in wave order.
    uint16_t* C = reinterpret_cast<uint16_t*>(p.c);
    for (int o = tid; o < nrb * CT * 256; o += (int)blockDim.x) {
        const int rbc = o >> 8, m = (o >> 4) & 15, n = o & 15;
        const int rb = rbc / CT, c = rbc % CT;
        const int row = rb * 16 + m;
        if (row >= rows) continue;
        const int sl = (n >> 2) * 16 + m, r = n & 3;
        float v = red[(rbc * nw) * 64 + sl][r];
        for (int w2 = 1; w2 < nw; ++w2) v += red[(rbc * nw + w2) * 64 + sl][r];
        const int64_t off = (int64_t)(row0 + row) * p.ldc + (tile0 + c) * 16 + n;
        store_up<DUAL>(C, p.c2, off, v);
    }
}

// Persistent variant of the chunk kernel (J = 8) for T >= kSkinnyStreamTokens.
// Workgroup (rank, s) visits the column tiles s, s + split, ... of its
// expert. The activation chunks of the expert's rows do not depend on the
// column, so they are loaded once and stay in registers; the weights of the
// next tile are requested before the current tile is multiplied, reduced and
// stored, so a workgroup's weight stream does not pause between tiles (two
// register sets alternate: a copy between them would wait for the loads).
// Lane/k assignment, MFMA order and wave order of the sums are the chunk
// kernel's, so the results are bit-identical to it. A past-the-end tile reads
// zeros from the buffer resource without touching memory.
//
// KS = 2 (GEMM_DOWN with K = 16 * 256 and more than 16 rows): K is split in
// two halves over twice the workgroups, (rank, s, half), so that 8 waves hold
// the rows of one half; each half's sums (wave order) are stored as fp32 rows
// of p.dpart and the combine adds the halves.
//
// Outputs are staged in LDS and written after the last tile. A global store
// inside the loop would be counted on the same in-order vector-memory counter
// as the weight loads issued before it, and the next register set's loads
// reuse the store's registers, so each tile boundary would wait for every
// outstanding load -- the prefetched tile included.
template <int KIND, bool DUAL, int RB, int KS>
__host__ __device__ constexpr int stream_stage_bytes() {  // staged outputs of one visited tile
    return 16 * RB * 16 * (KS == 2 ? 4 : 2) * (DUAL ? 2 : 1);
}
template <int KIND, bool DUAL, int RB, int NWMAX, int KS = 1>
__global__ __launch_bounds__(64 * NWMAX) void skinny_stream_kernel(GemmParams p, int nexp, int split) {
    static_assert(KIND == GEMM_UP || KIND == GEMM_DOWN, "forward GEMMs only");
    static_assert(KS == 1 || (KS == 2 && KIND == GEMM_DOWN && !DUAL), "K halves: GEMM_DOWN only");
    constexpr bool kGather = KIND == GEMM_UP;
    constexpr int J = 8;
    // [RB][nw][64] wave partials, then the staged outputs of each visited
    // tile: [16 RB rows][16 columns] fp32 (KS == 2) or bf16 C, then bf16
    // SiLU(C) when DUAL
    extern __shared__ f32x4 red[];
    __shared__ int s_tok[NWMAX][16 * RB];
    constexpr int TSB = stream_stage_bytes<KIND, DUAL, RB, KS>();

    const int nw = (int)blockDim.x >> 6;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rank = (int)blockIdx.x % nexp, sq = (int)blockIdx.x / nexp;
    const int s0 = KS == 1 ? sq : sq % split, half = KS == 1 ? 0 : sq / split;
    args_in_sgprs(p.order, p.offsets, p.idx, p.a, p.c, p.c2, p.E, p.N, p.slots, p.topk, p.lda, p.ldb, p.ldc);
    const bool self = p.self_dispatch != 0;
    int ent[kPickGroups];
    if (kGather || self) load_picks(p, lane, ent);
    const SkinnyExpert x = self ? self_expert(p, rank, ent) : skinny_expert(p, rank, lane);
    const int row0 = x.row0;
    const int rows = min(x.rows, 16 * RB);
    const int ntile = p.N >> 4;
    if (rows <= 0 || s0 >= ntile) return;
    const int nrb = (rows + 15) >> 4;
    const int g = lane >> 4, li = lane & 15;
    const int kw = half * nw * (32 * J) + wave * (32 * J) + g * 8;

    // The expert's weights [N][K] as one buffer (below 2 GiB: checked by the
    // host). The tile offset is a wave-uniform scalar offset and the lane
    // offsets are loop-invariant registers: an address register recomputed
    // per tile would be a write after the previous set's loads, and the
    // compiler waits for every outstanding load (the prefetched tile
    // included) before it. Past the last tile the loads go through an empty
    // resource (no records), which returns zeros without touching memory.
    const int wbytes = p.N * (int)p.ldb * 2;
    const __amdgpu_buffer_rsrc_t wr = weight_rsrc(x.w, wbytes);
    const __amdgpu_buffer_rsrc_t wr_none = weight_rsrc(x.w, 0);
    const int lane_off = (li * (int)p.ldb + kw) * 2;
    const int tile_bytes = 16 * (int)p.ldb * 2;
    auto wload = [&](int tile, uint4 (&w)[J]) {
        const bool in = tile < ntile;  // uniform
        const int soff = (in ? tile : ntile - 1) * tile_bytes;
#pragma unroll
        for (int i = 0; i < J; ++i)
            w[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(in ? wr : wr_none,
                                                                                   lane_off + 64 * i, soff, 0));
    };
    uint4 w0[J], w1[J];
    wload(s0, w0);

    const bool by_pick = kGather && p.idx != nullptr;
    if (by_pick) expert_tokens(ent, p.slots, p.topk, x.e, lane, 16 * RB, s_tok[wave]);
    uint4 av[RB][J];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int m = rb * 16 + li;
        const bool ok = m < rows;
        const int mm = ok ? m : 0;
        const int srow = by_pick ? s_tok[wave][mm] : row0 + mm;
        const uint16_t* ar = p.a + (int64_t)srow * p.lda + kw;
#pragma unroll
        for (int i = 0; i < J; ++i) av[rb][i] = (rb < nrb) ? ld16(ar + 32 * i) : make_uint4(0, 0, 0, 0);
        if (!ok) {
#pragma unroll
            for (int i = 0; i < J; ++i) av[rb][i] = make_uint4(0, 0, 0, 0);
        }
    }

    uint8_t* stage = reinterpret_cast<uint8_t*>(red + RB * nw * 64);
    auto step = [&](int tile, const uint4 (&w)[J]) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            if (rb >= nrb) break;  // uniform
            f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < J; ++i) acc = mfma16(w[i], av[rb][i], acc);
            red[(rb * nw + wave) * 64 + lane] = acc;
        }
        __syncthreads();
        uint8_t* st = stage + ((tile - s0) / split) * TSB;
        for (int o = tid; o < nrb * 256; o += (int)blockDim.x) {
            const int rb = o >> 8, m = (o >> 4) & 15, n = o & 15;
            const int row = rb * 16 + m;
            if (row >= rows) continue;
            const int sl = (n >> 2) * 16 + m, r = n & 3;
            float v = red[(rb * nw) * 64 + sl][r];
            for (int w2 = 1; w2 < nw; ++w2) v += red[(rb * nw + w2) * 64 + sl][r];
            if constexpr (KS == 2) {
                reinterpret_cast<float*>(st)[row * 16 + n] = v;
            } else {
                if constexpr (DUAL) {
                    float a, da;
                    silu_dsilu(v, a, da);
                    reinterpret_cast<uint16_t*>(st)[row * 16 + n] = f2bf(da);
                    reinterpret_cast<uint16_t*>(st)[16 * RB * 16 + row * 16 + n] = f2bf(a);
                } else {
                    reinterpret_cast<uint16_t*>(st)[row * 16 + n] = f2bf(v);
                }
            }
        }
        __syncthreads();
    };
    // The scheduling barriers keep the next tile's loads ahead of the
    // current tile's multiplies (the scheduler would otherwise sink them).
    for (int tile = s0; tile < ntile; tile += 2 * split) {
        wload(tile + split, w1);
        __builtin_amdgcn_sched_barrier(0);
        step(tile, w0);
        if (tile + split >= ntile) break;
        wload(tile + 2 * split, w0);
        __builtin_amdgcn_sched_barrier(0);
        step(tile + split, w1);
    }

    // Staged outputs to global memory, 16 bytes per store: a row of one tile
    // is 32 bytes of bf16 (two stores per plane) or 64 bytes of fp32 (four).
    constexpr int CPR = KS == 2 ? 4 : 2;  // 16-byte chunks per staged row
    constexpr int NPL = DUAL ? 2 : 1;     // output planes
    const int visited = (ntile - s0 + split - 1) / split;
    const int per_tile = rows * CPR * NPL;
    for (int o = tid; o < visited * per_tile; o += (int)blockDim.x) {
        const int j = o / per_tile, rem = o % per_tile;
        const int pl = rem / (rows * CPR), rc = rem % (rows * CPR);
        const int row = rc / CPR, c = rc % CPR;
        const int tile = s0 + j * split;
        const uint4 v = *reinterpret_cast<const uint4*>(stage + j * TSB + pl * (16 * RB * 16 * 2) +
                                                        (row * CPR + c) * 16);
        if constexpr (KS == 2) {
            *reinterpret_cast<uint4*>(p.dpart + ((int64_t)half * p.slots + row0 + row) * p.N + tile * 16 + c * 4) = v;
        } else {
            uint16_t* dst = pl == 0 ? reinterpret_cast<uint16_t*>(p.c) : p.c2;
            *reinterpret_cast<uint4*>(dst + (int64_t)(row0 + row) * p.ldc + tile * 16 + c * 8) = v;
        }
    }
}

template <int KIND, bool DUAL>
hipError_t launch_rb(int rb, const GemmParams& p, int nexp, unsigned grid, hipStream_t s) {
    switch (rb) {
        case 1: skinny_gemm_kernel<KIND, DUAL, 1><<<grid, kThreads, 0, s>>>(p, nexp); break;
        case 2: skinny_gemm_kernel<KIND, DUAL, 2><<<grid, kThreads, 0, s>>>(p, nexp); break;
        case 4: skinny_gemm_kernel<KIND, DUAL, 4><<<grid, kThreads, 0, s>>>(p, nexp); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int KIND, bool DUAL, int J, int CT>
hipError_t launch_chunk_rb(int rb, int nw, const GemmParams& p, int nexp, hipStream_t s) {
    const unsigned grid = (unsigned)(p.N / (16 * CT)) * (unsigned)nexp;
    const dim3 block(64 * nw);
    const size_t lds = (size_t)rb * CT * nw * 64 * sizeof(f32x4);
    switch (rb) {
        case 1: skinny_chunk_kernel<KIND, DUAL, J, 1, CT><<<grid, block, lds, s>>>(p, nexp, Route1{}); break;
        case 2: skinny_chunk_kernel<KIND, DUAL, J, 2, CT><<<grid, block, lds, s>>>(p, nexp, Route1{}); break;
        case 4: skinny_chunk_kernel<KIND, DUAL, J, 4, CT><<<grid, block, lds, s>>>(p, nexp, Route1{}); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
template <int KIND, bool DUAL>
hipError_t launch_chunk(int J, int ct, int rb, int nw, const GemmParams& p, int nexp, hipStream_t s) {
    if (ct == 2)
        return J == 8 ? launch_chunk_rb<KIND, DUAL, 8, 2>(rb, nw, p, nexp, s)
                      : launch_chunk_rb<KIND, DUAL, 2, 2>(rb, nw, p, nexp, s);
    return J == 8 ? launch_chunk_rb<KIND, DUAL, 8, 1>(rb, nw, p, nexp, s)
                  : launch_chunk_rb<KIND, DUAL, 2, 1>(rb, nw, p, nexp, s);
}

// Dynamic LDS of a stream-kernel workgroup: the wave partials and the staged
// outputs of every tile it visits (at most ceil(ntile / split)).
template <int KIND, bool DUAL, int RB, int KS>
size_t stream_lds(int nw, int ntile, int split) {
    return (size_t)RB * nw * 64 * sizeof(f32x4) +
           (size_t)((ntile + split - 1) / split) * stream_stage_bytes<KIND, DUAL, RB, KS>();
}
// Largest dynamic LDS the stream kernels take (beyond it the chunk kernel runs).
constexpr size_t kStreamMaxLds = 64 * 1024;

// GEMM_DOWN with K in two halves of 8 waves (rows of up to 64 tokens).
hipError_t launch_stream_halves(int rb, const GemmParams& p, int nexp, int split, hipStream_t s) {
    const unsigned grid = 2u * (unsigned)split * (unsigned)nexp;
    const dim3 block(64 * 8);
    const int ntile = p.N / 16;
    switch (rb) {
        case 2: skinny_stream_kernel<GEMM_DOWN, false, 2, 8, 2>
                    <<<grid, block, stream_lds<GEMM_DOWN, false, 2, 2>(8, ntile, split), s>>>(p, nexp, split); break;
        case 4: skinny_stream_kernel<GEMM_DOWN, false, 4, 8, 2>
                    <<<grid, block, stream_lds<GEMM_DOWN, false, 4, 2>(8, ntile, split), s>>>(p, nexp, split); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int KIND, bool DUAL>
hipError_t launch_stream(int rb, int nw, const GemmParams& p, int nexp, int split, hipStream_t s) {
    const unsigned grid = (unsigned)split * (unsigned)nexp;
    const dim3 block(64 * nw);
    const int ntile = p.N / 16;
    if (nw > 8) {
        if (rb != 1) return hipErrorInvalidValue;
        skinny_stream_kernel<KIND, DUAL, 1, 16>
            <<<grid, block, stream_lds<KIND, DUAL, 1, 1>(nw, ntile, split), s>>>(p, nexp, split);
        return hipGetLastError();
    }
    switch (rb) {
        case 1: skinny_stream_kernel<KIND, DUAL, 1, 8>
                    <<<grid, block, stream_lds<KIND, DUAL, 1, 1>(nw, ntile, split), s>>>(p, nexp, split); break;
        case 2: skinny_stream_kernel<KIND, DUAL, 2, 8>
                    <<<grid, block, stream_lds<KIND, DUAL, 2, 1>(nw, ntile, split), s>>>(p, nexp, split); break;
        case 4: skinny_stream_kernel<KIND, DUAL, 4, 8>
                    <<<grid, block, stream_lds<KIND, DUAL, 4, 1>(nw, ntile, split), s>>>(p, nexp, split); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
// Whether launch_stream's workgroups fit kStreamMaxLds.
size_t stream_lds_rt(bool halves, bool dual, int rb, int nw, int ntile, int split) {
    if (halves) return rb == 2 ? stream_lds<GEMM_DOWN, false, 2, 2>(nw, ntile, split)
                               : stream_lds<GEMM_DOWN, false, 4, 2>(nw, ntile, split);
    switch (rb) {
        case 1: return dual ? stream_lds<GEMM_UP, true, 1, 1>(nw, ntile, split) : stream_lds<GEMM_UP, false, 1, 1>(nw, ntile, split);
        case 2: return dual ? stream_lds<GEMM_UP, true, 2, 1>(nw, ntile, split) : stream_lds<GEMM_UP, false, 2, 1>(nw, ntile, split);
        default: return dual ? stream_lds<GEMM_UP, true, 4, 1>(nw, ntile, split) : stream_lds<GEMM_UP, false, 4, 1>(nw, ntile, split);
    }
}


}  // namespace

// Compute units of the current device (cached per device).
int cu_count() {
    static int cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

namespace {

// Launch shape of the skinny kernels for a reduction length K.
struct SkinnyShape {
    int J = 0, nw = 0;  // MFMAs per wave chunk (8 or 2, 0: neither) and waves
    int rb = 1;         // 16-row blocks held per workgroup
};
SkinnyShape skinny_shape(int K, int T) {
    SkinnyShape sh;
    // One K-chunk per wave, at most 16 waves.
    if (K % 256 == 0 && K / 256 >= 4 && K / 256 <= 16) {
        sh.J = 8;
        sh.nw = K / 256;
    } else if (K / 64 <= 16) {
        sh.J = 2;
        sh.nw = K / 64;
    }
    sh.rb = T <= 16 ? 1 : (T <= 32 ? 2 : 4);
    return sh;
}
// Workgroups per expert of the stream kernel, or 0 where it does not apply:
// persistent workgroups where the activation chunks fit in registers next to
// two weight sets (up to 8 waves for any row count, 16 waves for one row
// block) and the staged outputs fit kStreamMaxLds.
int stream_split(const SkinnyShape& sh, int T, int N, int64_t ldb, int nexp, bool dual) {
    if (sh.J != 8 || T < kSkinnyStreamTokens || !(sh.nw <= 8 || sh.rb == 1) || (int64_t)N * ldb * 2 >= (1ll << 31))
        return 0;
    const int ntile = N / 16;
    const int per_cu = sh.nw > 8 ? 1 : (sh.rb == 4 ? 2 : (sh.rb == 2 ? 3 : 4)) * 4 / sh.nw;
    int split = (cu_count() * (per_cu > 0 ? per_cu : 1) + nexp - 1) / nexp;
    split = split < 1 ? 1 : (split > ntile ? ntile : split);
    return stream_lds_rt(false, dual, sh.rb, sh.nw, ntile, split) <= kStreamMaxLds ? split : 0;
}
// Workgroups per expert and K half of GEMM_DOWN over 16 waves with more than
// one row block (two K halves of 8 waves each keep the rows resident, one
// 8-wave workgroup per CU), or 0 where it does not apply.
int halves_split(const SkinnyShape& sh, int T, int N, int64_t ldb, int nexp) {
    if (sh.J != 8 || sh.nw != 16 || sh.rb <= 1 || T < kSkinnyStreamTokens || (int64_t)N * ldb * 2 >= (1ll << 31))
        return 0;
    const int ntile = N / 16;
    int split = (cu_count() + 2 * nexp - 1) / (2 * nexp);
    split = split < 1 ? 1 : (split > ntile ? ntile : split);
    return stream_lds_rt(true, false, sh.rb, 8, ntile, split) <= kStreamMaxLds ? split : 0;
}

}  // namespace

bool skinny_up_route1_fits(int d, int E) {
    const SkinnyShape sh = skinny_shape(d, 1);
    return E > 1 && E <= kMaxExperts && (sh.J == 8 || sh.J == 2) && sh.nw >= 1;
}

hipError_t launch_skinny_up_route1(bool dual, const GemmParams& p, const Route1& r, hipStream_t s) {
    if (!skinny_up_route1_fits(p.K, p.E) || p.N % 16 != 0 || p.N <= 0 || r.rp.T != 1 || r.rp.d != p.K ||
        r.rp.E != p.E || r.rp.K != p.topk || p.slots != p.topk || p.topk > kMaxTopK)
        return hipErrorInvalidValue;
    const SkinnyShape sh = skinny_shape(p.K, 1);
    const int nexp = p.topk;  // one rank per pick
    const unsigned grid = (unsigned)(p.N / 16) * (unsigned)nexp;
    const dim3 block(64 * sh.nw);
    const size_t lds = (size_t)sh.nw * 64 * sizeof(f32x4);
#define TMT_R1(EP_)                                                                                       \
    case EP_:                                                                                            \
        if (sh.J == 8) {                                                                                 \
            if (dual) skinny_chunk_kernel<GEMM_UP, true, 8, 1, 1, EP_><<<grid, block, lds, s>>>(p, nexp, r); \
            else skinny_chunk_kernel<GEMM_UP, false, 8, 1, 1, EP_><<<grid, block, lds, s>>>(p, nexp, r);     \
        } else {                                                                                         \
            if (dual) skinny_chunk_kernel<GEMM_UP, true, 2, 1, 1, EP_><<<grid, block, lds, s>>>(p, nexp, r); \
            else skinny_chunk_kernel<GEMM_UP, false, 2, 1, 1, EP_><<<grid, block, lds, s>>>(p, nexp, r);     \
        }                                                                                                \
        break;
    switch (router_ep(p.E)) {
        TMT_R1(8)
        TMT_R1(16)
        TMT_R1(32)
        TMT_R1(64)
        default: return hipErrorInvalidValue;
    }
#undef TMT_R1
    return hipGetLastError();
}

bool skinny_self_dispatch(int T, int E, int K, int d, int h, int hn) {
    (void)K;
    if (E <= 1 || T <= 1 || T > kSkinnyMaxTokens || hn % 16 != 0 || d % 64 != 0 || h % 64 != 0) return false;
    if (stream_split(skinny_shape(d, T), T, hn, d, E, h > 0) == 0) return false;
    if (h == 0) return true;
    // GEMM_DOWN: the stream kernel, or its K halves
    const SkinnyShape sh = skinny_shape(h, T);
    if (stream_split(sh, T, d, h, E, false) > 0) return true;
    return halves_split(sh, T, d, h, E) > 0;
}

hipError_t launch_skinny_gemm(GemmKind kind, bool dual, const GemmParams& p, int T, hipStream_t s,
                              bool* halves) {
    if (halves != nullptr) *halves = false;
    if (T <= 0) return hipSuccess;
    if (T > kSkinnyMaxTokens || p.N % 16 != 0 || p.K % 64 != 0 || p.N <= 0) return hipErrorInvalidValue;
    if (kind != GEMM_UP && kind != GEMM_DOWN) return hipErrorInvalidValue;
    const bool self = p.self_dispatch != 0;
    // Ranks of the grid: experts in processing order, at most one per pick;
    // self_dispatch indexes the grid by expert (empty experts exit at once).
    const int nexp = self ? p.E : min(p.E, p.slots);
    const SkinnyShape sh = skinny_shape(p.K, T);
    const int J = sh.J, nw = sh.nw, rb = sh.rb;
    const int split = stream_split(sh, T, p.N, p.ldb, nexp, kind == GEMM_UP && dual);
    if (split > 0) {
        if (kind == GEMM_UP)
            return dual ? launch_stream<GEMM_UP, true>(rb, nw, p, nexp, split, s)
                        : launch_stream<GEMM_UP, false>(rb, nw, p, nexp, split, s);
        return launch_stream<GEMM_DOWN, false>(rb, nw, p, nexp, split, s);
    }
    if (kind == GEMM_DOWN && p.dpart != nullptr && halves != nullptr) {
        const int hs = halves_split(sh, T, p.N, p.ldb, nexp);
        if (hs > 0) {
            *halves = true;
            return launch_stream_halves(rb, p, nexp, hs, s);
        }
    }
    if (self) return hipErrorInvalidValue;  // the host checked skinny_self_dispatch
    if (J > 0) {
        const int ct = (T >= kSkinnyTwoTileTokens && p.N % 32 == 0) ? 2 : 1;
        if (kind == GEMM_UP)
            return dual ? launch_chunk<GEMM_UP, true>(J, ct, rb, nw, p, nexp, s)
                        : launch_chunk<GEMM_UP, false>(J, ct, rb, nw, p, nexp, s);
        return launch_chunk<GEMM_DOWN, false>(J, ct, rb, nw, p, nexp, s);
    }
    // General reduction lengths: K split over 4 waves in 64-element units.
    const unsigned grid = (unsigned)(p.N / 16) * (unsigned)nexp;
    if (kind == GEMM_UP)
        return dual ? launch_rb<GEMM_UP, true>(rb, p, nexp, grid, s)
                    : launch_rb<GEMM_UP, false>(rb, p, nexp, grid, s);
    return launch_rb<GEMM_DOWN, false>(rb, p, nexp, grid, s);
}

}  // namespace tmt

// ------------------------------------------------ one-token down + combine --
namespace tmt {
namespace {

__device__ __forceinline__ float bf16_to_float(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }

// One token, K experts: O_j = W_down[e_j] . a_j for the 4 columns of this
// workgroup, then Y = beta * Y + sum_j gate_j * bf16(O_j) (the combine's
// expression and pick order). Wave w reduces k in [256 w, 256 w + 256); lane
// half hf covers rows hf, hf + 2, ... of the 4K (pick, column) rows with 8
// consecutive k per lane; each half-wave adds its 32 lanes by a butterfly
// and the waves are added in order through LDS.
template <int K>
__global__ __launch_bounds__(1024) void down_combine1_kernel(Down1Params p) {
    constexpr int R = 4 * K, RH = R / 2;  // (pick, column) rows; per lane half
    __shared__ float part[16][R];
    __shared__ float o_s[R];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nw = (int)blockDim.x >> 6;
    const int n0 = (int)blockIdx.x * 4;
    const int hf = lane >> 5, sub = lane & 31;
    const int k0 = wave * 256 + sub * 8;
    // the token's picks (one round trip), then everything that depends on them
    int e[K], sl[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
        e[j] = __builtin_amdgcn_readfirstlane(p.idx[j]);
        sl[j] = __builtin_amdgcn_readfirstlane(p.slot_of[j]);
    }
    uint4 wv[RH], av[K];
#pragma unroll
    for (int q = 0; q < RH; ++q) {
        const int r = 2 * q + hf, j = r >> 2, c = r & 3;
        wv[q] = *reinterpret_cast<const uint4*>(p.w[e[j]] + (int64_t)(n0 + c) * p.h + k0);
    }
#pragma unroll
    for (int j = 0; j < K; ++j) av[j] = *reinterpret_cast<const uint4*>(p.a + (int64_t)sl[j] * p.h + k0);
    float acc[RH];
#pragma unroll
    for (int q = 0; q < RH; ++q) {
        const int j = (2 * q + hf) >> 2;
        float wf[8], af[8];
        unpack8(wv[q], wf);
        unpack8(av[j], af);
        float s = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; ++t) s = __builtin_fmaf(wf[t], af[t], s);
        acc[q] = s;
    }
#pragma unroll
    for (int q = 0; q < RH; ++q) {
        float v = acc[q];
        v += __shfl_xor(v, 16, 64);
        v += __shfl_xor(v, 8, 64);
        v += __shfl_xor(v, 4, 64);
        v += __shfl_xor(v, 2, 64);
        v += __shfl_xor(v, 1, 64);
        if (sub == 0) part[wave][2 * q + hf] = v;
    }
    __syncthreads();
    if (tid < R) {
        float v = part[0][tid];
        for (int w2 = 1; w2 < nw; ++w2) v += part[w2][tid];
        const uint16_t ob = f2bf(v);
        const int j = tid >> 2, c = tid & 3;
        p.O[(int64_t)sl[j] * p.d + n0 + c] = ob;
        o_s[tid] = bf16_to_float(ob);
    }
    __syncthreads();
    if (tid < 4) {
        float y = p.beta != 0.0f ? bf16_to_float(p.Y[n0 + tid]) * p.beta : 0.0f;
#pragma unroll
        for (int j = 0; j < K; ++j) y += p.gate[j] * o_s[4 * j + tid];
        p.Y[n0 + tid] = f2bf(y);
    }
}

}  // namespace

bool decode1_down_combine_fits(int d, int h, int K) {
    return K >= 1 && K <= 8 && h % 256 == 0 && h / 256 >= 4 && h / 256 <= 16 && d % 4 == 0 && d > 0;
}

hipError_t launch_decode1_down_combine(const Down1Params& p, hipStream_t s) {
    if (!decode1_down_combine_fits(p.d, p.h, p.K)) return hipErrorInvalidValue;
    const dim3 grid(p.d / 4), block(64 * (p.h / 256));
    switch (p.K) {
#define TMT_D1(KK) case KK: down_combine1_kernel<KK><<<grid, block, 0, s>>>(p); break;
        TMT_D1(1) TMT_D1(2) TMT_D1(3) TMT_D1(4) TMT_D1(5) TMT_D1(6) TMT_D1(7) TMT_D1(8)
#undef TMT_D1
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace tmt
