// moe_oracle.cpp -- CPU restatement of TMT's MoE block (test infrastructure).
//
// TEST INFRASTRUCTURE ONLY: this file is the parity checker for the HIP
// library. Nothing in the product path may call it. Build: oracle/Makefile
// (g++ -O3 -ffp-contract=off; contraction would change the canonical router
// sums). Reference citations are relative to the reference tree.
#include "moe_oracle.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <functional>
#include <limits>
#include <thread>
#include <vector>

namespace {

inline float bf(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// Round to nearest even; NaN stays NaN (quieted). Same rule as the
// reference's __float2bfloat16_rn (tmt-cuda/src/common.h:12-14).
inline uint16_t tobf(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// common.h:15-24: sigmoid = 1/(1+exp(-x)); silu = x*sigmoid;
// silu_bwd(x, g) = g*s*(1 + x*(1-s)). Evaluated in double, rounded once.
inline float silu_f(float x) { return (float)((double)x / (1.0 + std::exp(-(double)x))); }
inline float dsilu_f(float x) {
    double s = 1.0 / (1.0 + std::exp(-(double)x));
    return (float)(s * (1.0 + (double)x * (1.0 - s)));
}

int nthreads(int requested) {
    if (requested > 0) return requested;
    unsigned hc = std::thread::hardware_concurrency();
    return hc ? (int)hc : 1;
}

// Runs fn(task) for task in [0, n). Each task owns disjoint outputs, so the
// result does not depend on which thread ran it.
void run_tasks(int64_t n, int threads, const std::function<void(int64_t)>& fn) {
    threads = (int)std::min<int64_t>(nthreads(threads), std::max<int64_t>(n, 1));
    if (threads <= 1) {
        for (int64_t i = 0; i < n; ++i) fn(i);
        return;
    }
    std::atomic<int64_t> next{0};
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; ++t)
        pool.emplace_back([&] {
            for (int64_t i; (i = next.fetch_add(1)) < n;) fn(i);
        });
    for (auto& th : pool) th.join();
}

// C[m][0:N] = sum_k A(m)[k] * B[k][0:N] for m in [0, M); A rows by pointer.
// Blocked over 8 rows x 512 columns; the k loop runs in ascending order.
void gemm_rows(int64_t M, int N, int K, const float* const* arow,
               const float* B, int64_t ldb, float* C, int64_t ldc, int threads) {
    const int MB = 8, NB = 512;
    int64_t mblocks = (M + MB - 1) / MB;
    int64_t nblocks = (N + NB - 1) / NB;
    run_tasks(mblocks * nblocks, threads, [&](int64_t task) {
        int64_t m0 = (task / nblocks) * MB;
        int n0 = (int)(task % nblocks) * NB;
        int mb = (int)std::min<int64_t>(MB, M - m0);
        int nb = std::min(NB, N - n0);
        float acc[MB][NB];
        for (int i = 0; i < mb; ++i) std::fill(acc[i], acc[i] + nb, 0.0f);
        for (int k = 0; k < K; ++k) {
            const float* brow = B + (int64_t)k * ldb + n0;
            for (int i = 0; i < mb; ++i) {
                float a = arow[m0 + i][k];
                if (a == 0.0f) continue;
                float* c = acc[i];
                for (int n = 0; n < nb; ++n) c[n] += a * brow[n];
            }
        }
        for (int i = 0; i < mb; ++i)
            std::memcpy(C + (m0 + i) * ldc + n0, acc[i], sizeof(float) * nb);
    });
}

// dst[c][r] = src[r][c] for an R x Cn fp32 matrix.
void transpose(const float* src, int64_t R, int64_t Cn, int64_t lds, float* dst) {
    for (int64_t r = 0; r < R; ++r)
        for (int64_t c = 0; c < Cn; ++c) dst[c * R + r] = src[r * lds + c];
}

std::vector<float> to_f32(const uint16_t* p, int64_t n) {
    std::vector<float> v(n);
    for (int64_t i = 0; i < n; ++i) v[i] = bf(p[i]);
    return v;
}

bool dims_ok(const orc_dims* dm) {
    if (!dm) return false;
    if (dm->T < 0 || dm->d <= 0 || dm->E < 1 || dm->K < 1 || dm->K > dm->E || dm->h < 0) return false;
    if (dm->E == 1 && dm->K != 1) return false;
    return true;
}

// Everything the backward needs from the forward.
struct Fwd {
    std::vector<float> logits, probs, w, lse, Xf, U, A, O;
    std::vector<int32_t> idx, counts, offsets, perm, slot_of;
    float aux = 0, z = 0;
};

float canonical_logit(const uint16_t* x, const uint16_t* w, int d) {
    // Canonical fp32 order (the GPU router reproduces it bit for bit):
    // element k goes to lane L = (k/8) mod 64; each lane accumulates its
    // elements in ascending k with fmaf starting from +0; the 64 lane sums
    // are combined by an xor butterfly with offsets 32,16,8,4,2,1
    // (v[i] <- v[i] + v[i^off]; addition is commutative, so every lane ends
    // with the same value). This replaces the reference's 8-lanes-per-expert
    // shuffle tree (tmt-cuda/src/moe.cu:21-38), whose exact order cannot be
    // reproduced for E > 8 (it is undefined there).
    float lane[64];
    for (int i = 0; i < 64; ++i) lane[i] = 0.0f;
    for (int k = 0; k < d; ++k) {
        int L = (k >> 3) & 63;
        lane[L] = std::fma(bf(x[k]), bf(w[k]), lane[L]);
    }
    for (int off = 32; off >= 1; off >>= 1) {
        float nv[64];
        for (int i = 0; i < 64; ++i) nv[i] = lane[i] + lane[i ^ off];
        std::memcpy(lane, nv, sizeof(lane));
    }
    return lane[0];
}

// LayerNorm row statistics in the canonical order shared with the GPU kernel
// (the lane layout of canonical_logit): element k goes to lane (k/8) mod 64;
// each lane adds its elements (sum) and accumulates x*x with fmaf (sum of
// squares) in ascending k from +0; an xor butterfly 32..1 combines the lanes.
// mean = sum/D, var = sumsq/D - mean*mean, rstd = 1/sqrt(var + 1e-5), each
// operation rounded on its own (tmt-cuda/src/norm.cu:13-44, whose block-tree
// order and rsqrtf are replaced by this order and IEEE sqrt / division).
void ln_row_stats(const uint16_t* x, int d, float* mean, float* rstd) {
    float ls[64], lq[64];
    for (int i = 0; i < 64; ++i) ls[i] = lq[i] = 0.0f;
    for (int k = 0; k < d; ++k) {
        const int L = (k >> 3) & 63;
        const float v = bf(x[k]);
        ls[L] = ls[L] + v;
        lq[L] = std::fma(v, v, lq[L]);
    }
    for (int off = 32; off >= 1; off >>= 1) {
        float ns[64], nq[64];
        for (int i = 0; i < 64; ++i) {
            ns[i] = ls[i] + ls[i ^ off];
            nq[i] = lq[i] + lq[i ^ off];
        }
        std::memcpy(ls, ns, sizeof(ls));
        std::memcpy(lq, nq, sizeof(lq));
    }
    const float m = ls[0] / (float)d;
    const float qd = lq[0] / (float)d;
    const float m2 = m * m;
    const float var = qd - m2;
    *mean = m;
    *rstd = 1.0f / std::sqrt(var + 1e-5f);
}

void router_rows(const orc_dims* dm, const uint16_t* X, const uint16_t* Wr,
                 const float* bias, float* logits, float* probs, int32_t* idx,
                 float* w, float* lse) {
    const int T = dm->T, d = dm->d, E = dm->E, K = dm->K;
    run_tasks((T + 63) / 64, dm->threads, [&](int64_t blk) {
        int r0 = (int)blk * 64, r1 = std::min(T, r0 + 64);
        std::vector<float> l(E);
        std::vector<char> used(E);
        for (int r = r0; r < r1; ++r) {
            const uint16_t* x = X + (int64_t)r * d;
            for (int e = 0; e < E; ++e) {
                float v = canonical_logit(x, Wr + (int64_t)e * d, d);
                if (bias) v = v + bias[e];
                l[e] = v;
            }
            // Softmax (moe.cu:41-49 / :77-81), evaluated in double.
            double mx = l[0];
            for (int e = 1; e < E; ++e) mx = std::max(mx, (double)l[e]);
            double se = 0;
            for (int e = 0; e < E; ++e) se += std::exp((double)l[e] - mx);
            std::vector<double> p(E);
            for (int e = 0; e < E; ++e) p[e] = std::exp((double)l[e] - mx) / se;
            // Top-k (moe.cu:82-91): first maximum over ascending e with a strict
            // '>' (ties -> lower index). Applied to logits, which order the
            // experts exactly as the exact probabilities do.
            std::fill(used.begin(), used.end(), 0);
            double zs = 0;
            int sel[64];
            for (int j = 0; j < K; ++j) {
                int best = -1;
                float bv = 0;
                for (int e = 0; e < E; ++e) {
                    if (used[e]) continue;
                    if (best < 0 || l[e] > bv) { best = e; bv = l[e]; }
                }
                used[best] = 1;
                sel[j] = best;
                zs += (double)(float)p[best];
            }
            for (int e = 0; e < E; ++e) {
                if (logits) logits[(int64_t)r * E + e] = l[e];
                if (probs) probs[(int64_t)r * E + e] = (float)p[e];
            }
            for (int j = 0; j < K; ++j) {
                if (idx) idx[(int64_t)r * K + j] = sel[j];
                // Renormalised gate (moe.cu:92-94).
                if (w) w[(int64_t)r * K + j] = (float)((double)(float)p[sel[j]] / zs);
            }
            if (lse) lse[r] = (float)(mx + std::log(se));
        }
    });
}

void dispatch(int T, int E, int K, const int32_t* idx, int32_t* counts,
              int32_t* offsets, int32_t* perm, int32_t* slot_of) {
    // count_kernel (moe.cu:97-101) + exclusive scan (moe.cu:412-413) +
    // fill_kernel (moe.cu:103-115) with the canonical stable order: inside an
    // expert segment, slots follow ascending token index.
    std::vector<int32_t> cnt(E, 0), cur(E + 1, 0);
    for (int64_t i = 0; i < (int64_t)T * K; ++i) cnt[idx[i]]++;
    for (int e = 0; e < E; ++e) cur[e + 1] = cur[e] + cnt[e];
    if (counts) std::copy(cnt.begin(), cnt.end(), counts);
    if (offsets) std::copy(cur.begin(), cur.end(), offsets);
    for (int r = 0; r < T; ++r)
        for (int j = 0; j < K; ++j) {
            int e = idx[(int64_t)r * K + j];
            int pos = cur[e]++;
            if (perm) perm[pos] = r;
            if (slot_of) slot_of[(int64_t)r * K + j] = pos;
        }
}

void aux_z(int T, int E, int K, const float* probs, const int32_t* counts,
           const float* lse, float* aux, float* z) {
    // aux = E * sum_e (sum_r p_re / T) * (cnt_e / (T*K))   (moe.cu:453-465)
    // z   = (1/T) * sum_r lse_r^2                          (moe.cu:268-278)
    double a = 0, zz = 0;
    if (T > 0) {
        for (int e = 0; e < E; ++e) {
            double sp = 0;
            for (int r = 0; r < T; ++r) sp += probs[(int64_t)r * E + e];
            a += (sp / T) * ((double)counts[e] / ((double)T * K));
        }
        for (int r = 0; r < T; ++r) zz += (double)lse[r] * lse[r];
        zz /= T;
    }
    if (aux) *aux = (float)(E * a);
    if (z) *z = (float)zz;
}

// Forward into `f`. Keeps U (pre-activation), A = silu(U) and O.
int forward_impl(const orc_dims* dm, const uint16_t* X, const uint16_t* Wr,
                 const float* bias, const uint16_t* const* W_up,
                 const uint16_t* const* W_down, Fwd& f) {
    const int T = dm->T, d = dm->d, E = dm->E, K = dm->K, h = dm->h;
    const int hn = h > 0 ? h : d;  // width of the first expert GEMM
    const int64_t TK = (int64_t)T * K;
    f.Xf = to_f32(X, (int64_t)T * d);
    f.idx.assign(TK, 0);
    f.w.assign(TK, 1.0f);
    f.counts.assign(E, 0);
    f.offsets.assign(E + 1, 0);
    f.perm.assign(TK, 0);
    f.slot_of.assign(TK, 0);
    if (E > 1) {
        f.logits.assign((int64_t)T * E, 0);
        f.probs.assign((int64_t)T * E, 0);
        f.lse.assign(T, 0);
        router_rows(dm, X, Wr, bias, f.logits.data(), f.probs.data(),
                    f.idx.data(), f.w.data(), f.lse.data());
        dispatch(T, E, K, f.idx.data(), f.counts.data(), f.offsets.data(),
                 f.perm.data(), f.slot_of.data());
        aux_z(T, E, K, f.probs.data(), f.counts.data(), f.lse.data(), &f.aux, &f.z);
    } else {
        // E == 1: dense path without router (moe.cu:397-403).
        f.counts[0] = T;
        f.offsets[1] = T;
        for (int r = 0; r < T; ++r) { f.perm[r] = r; f.slot_of[r] = r; }
    }
    f.U.assign(TK * hn, 0.0f);
    if (h > 0) {
        f.A.assign(TK * h, 0.0f);
        f.O.assign(TK * d, 0.0f);
    }
    for (int e = 0; e < E; ++e) {
        int64_t s0 = f.offsets[e], cnt = f.offsets[e + 1] - s0;
        if (cnt == 0) continue;
        // Up / single linear: U = Xg * W^T with W [hn][d] ([out,in],
        // linalg.cu:9-17). Transpose W once so the inner loop is contiguous.
        std::vector<float> Wf = to_f32(W_up[e], (int64_t)hn * d), WT((int64_t)d * hn);
        transpose(Wf.data(), hn, d, d, WT.data());
        std::vector<const float*> rows(cnt);
        for (int64_t m = 0; m < cnt; ++m) rows[m] = f.Xf.data() + (int64_t)f.perm[s0 + m] * d;
        gemm_rows(cnt, hn, d, rows.data(), WT.data(), hn, f.U.data() + s0 * hn, hn, dm->threads);
        if (h > 0) {
            for (int64_t i = s0 * h; i < (s0 + cnt) * h; ++i) f.A[i] = silu_f(f.U[i]);
            std::vector<float> Df = to_f32(W_down[e], (int64_t)d * h), DT((int64_t)h * d);
            transpose(Df.data(), d, h, h, DT.data());
            for (int64_t m = 0; m < cnt; ++m) rows[m] = f.A.data() + (s0 + m) * h;
            gemm_rows(cnt, d, h, rows.data(), DT.data(), d, f.O.data() + s0 * d, d, dm->threads);
        }
    }
    return 0;
}

void combine(const orc_dims* dm, const Fwd& f, const uint16_t* Y_in, float beta, float* Y_out) {
    // combine_kernel (moe.cu:142-158): y = beta*y + sum_j w_j * expert_j.
    // In h == 0 mode SiLU is applied here, as in the reference.
    const int T = dm->T, d = dm->d, K = dm->K, h = dm->h;
    run_tasks(T, dm->threads, [&](int64_t r) {
        for (int c = 0; c < d; ++c) {
            float acc = (beta != 0.0f && Y_in) ? beta * bf(Y_in[r * d + c]) : 0.0f;
            for (int j = 0; j < K; ++j) {
                int64_t pos = f.slot_of[r * K + j];
                float v = h > 0 ? f.O[pos * d + c] : silu_f(f.U[pos * d + c]);
                acc += f.w[r * K + j] * v;
            }
            Y_out[r * d + c] = acc;
        }
    });
}

void router_bwd_rows(int T, int E, int K, const float* probs, const int32_t* idx,
                     const float* s, const float* lse_or_null, const float* logits,
                     const int32_t* counts, float aux_coef, float z_coef, float* dl) {
    // router_bwd_kernel (moe.cu:199-234), evaluated in double per row.
    for (int r = 0; r < T; ++r) {
        const float* p = probs + (int64_t)r * E;
        double Z = 0, sp = 0;
        for (int j = 0; j < K; ++j) {
            double pj = p[idx[(int64_t)r * K + j]];
            Z += pj;
            sp += (double)s[(int64_t)r * K + j] * pj;
        }
        double Z2 = Z * Z + 1e-12;
        std::vector<double> g(E, 0.0);
        for (int j = 0; j < K; ++j)
            g[idx[(int64_t)r * K + j]] = ((double)s[(int64_t)r * K + j] * Z - sp) / Z2;
        double acc = 0, expected = 0;
        for (int e = 0; e < E; ++e) {
            acc += g[e] * p[e];
            expected += (double)p[e] * counts[e] / ((double)T * K);
        }
        double lse;
        if (lse_or_null) {
            lse = lse_or_null[r];
        } else {
            const float* l = logits + (int64_t)r * E;
            double mx = l[0];
            for (int e = 1; e < E; ++e) mx = std::max(mx, (double)l[e]);
            double se = 0;
            for (int e = 0; e < E; ++e) se += std::exp((double)l[e] - mx);
            lse = mx + std::log(se);
        }
        for (int e = 0; e < E; ++e) {
            double v = p[e] * (g[e] - acc);
            v += (double)aux_coef * E / T * p[e] * ((double)counts[e] / ((double)T * K) - expected);
            v += (double)z_coef * 2.0 / T * lse * p[e];
            dl[(int64_t)r * E + e] = (float)v;
        }
    }
}

}  // namespace

extern "C" {

void orc_f32_to_bf16(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = tobf(in[i]);
}
void orc_bf16_to_f32(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = bf(in[i]);
}

float orc_router_logit(const uint16_t* x, const uint16_t* w, int32_t d) {
    return canonical_logit(x, w, d);
}

int orc_router(const orc_dims* dm, const uint16_t* X, const uint16_t* Wr,
               const float* bias, float* logits, float* probs, int32_t* idx,
               float* w, float* lse) {
    if (!dims_ok(dm) || !X || !Wr) return -1;
    router_rows(dm, X, Wr, bias, logits, probs, idx, w, lse);
    return 0;
}

int orc_dispatch(const orc_dims* dm, const int32_t* idx, int32_t* counts,
                 int32_t* offsets, int32_t* perm, int32_t* slot_of) {
    if (!dims_ok(dm) || !idx) return -1;
    for (int64_t i = 0; i < (int64_t)dm->T * dm->K; ++i)
        if (idx[i] < 0 || idx[i] >= dm->E) return -2;
    dispatch(dm->T, dm->E, dm->K, idx, counts, offsets, perm, slot_of);
    return 0;
}

int orc_aux_z(const orc_dims* dm, const float* probs, const int32_t* counts,
              const float* lse, float* aux, float* z) {
    if (!dims_ok(dm) || !probs || !counts || !lse) return -1;
    aux_z(dm->T, dm->E, dm->K, probs, counts, lse, aux, z);
    return 0;
}

int orc_forward(const orc_dims* dm, const uint16_t* X, const uint16_t* Wr,
                const float* bias, const uint16_t* const* W_up,
                const uint16_t* const* W_down, const uint16_t* Y_in,
                float beta, float* Y_out, float* logits, float* probs,
                int32_t* idx, float* w, int32_t* counts, int32_t* offsets,
                int32_t* perm, int32_t* slot_of, float* aux, float* z) {
    if (!dims_ok(dm) || !X || !W_up || !Y_out) return -1;
    if (dm->E > 1 && !Wr) return -1;
    if (dm->h > 0 && !W_down) return -1;
    Fwd f;
    int rc = forward_impl(dm, X, Wr, bias, W_up, W_down, f);
    if (rc) return rc;
    combine(dm, f, Y_in, beta, Y_out);
    const int64_t T = dm->T, E = dm->E, K = dm->K;
    if (E > 1) {
        if (logits) std::copy(f.logits.begin(), f.logits.end(), logits);
        if (probs) std::copy(f.probs.begin(), f.probs.end(), probs);
    }
    if (idx) std::copy(f.idx.begin(), f.idx.end(), idx);
    if (w) std::copy(f.w.begin(), f.w.end(), w);
    if (counts) std::copy(f.counts.begin(), f.counts.end(), counts);
    if (offsets) std::copy(f.offsets.begin(), f.offsets.end(), offsets);
    if (perm) std::copy(f.perm.begin(), f.perm.begin() + T * K, perm);
    if (slot_of) std::copy(f.slot_of.begin(), f.slot_of.end(), slot_of);
    if (aux) *aux = f.aux;
    if (z) *z = f.z;
    return 0;
}

int orc_backward(const orc_dims* dm, const uint16_t* X, const uint16_t* Wr,
                 const float* bias, const uint16_t* const* W_up,
                 const uint16_t* const* W_down, const uint16_t* dY,
                 float aux_coef, float z_coef, float* dX, float* dWr,
                 float* const* dW_up, float* const* dW_down) {
    if (!dims_ok(dm) || !X || !W_up || !dY || !dX || !dW_up) return -1;
    if (dm->E > 1 && (!Wr || !dWr)) return -1;
    if (dm->h > 0 && (!W_down || !dW_down)) return -1;
    const int T = dm->T, d = dm->d, E = dm->E, K = dm->K, h = dm->h;
    const int hn = h > 0 ? h : d;
    const int64_t TK = (int64_t)T * K;
    Fwd f;
    int rc = forward_impl(dm, X, Wr, bias, W_up, W_down, f);
    if (rc) return rc;
    std::vector<float> dYf = to_f32(dY, (int64_t)T * d);

    // Combine backward (moe.cu:160-197): s_rj = dY_r . expert_j(x_r); the
    // expert-output gradient is w_rj * dY_r (h > 0) or w*silu'(U)*dY (h == 0).
    std::vector<float> s(TK, 0.0f), dOut(TK * (h > 0 ? d : hn), 0.0f);
    run_tasks(T, dm->threads, [&](int64_t r) {
        const float* dy = dYf.data() + r * d;
        for (int j = 0; j < K; ++j) {
            int64_t pos = f.slot_of[r * K + j];
            float wj = f.w[r * K + j];
            double acc = 0;
            for (int c = 0; c < d; ++c) {
                float u = h > 0 ? f.O[pos * d + c] : f.U[pos * d + c];
                float v = h > 0 ? u : silu_f(u);
                acc += (double)dy[c] * v;
                dOut[pos * d + c] = h > 0 ? wj * dy[c] : wj * dy[c] * dsilu_f(u);
            }
            s[r * K + j] = (float)acc;
        }
    });

    // Router backward (moe.cu:199-234) then dWr = dl^T X (moe.cu:521) and the
    // router part of dX = dl * Wr (moe.cu:522-531), both fp32 here.
    std::vector<float> dl;
    if (E > 1) {
        dl.assign((int64_t)T * E, 0.0f);
        router_bwd_rows(T, E, K, f.probs.data(), f.idx.data(), s.data(), f.lse.data(),
                        nullptr, f.counts.data(), aux_coef, z_coef, dl.data());
        std::vector<float> dlT((int64_t)E * T);
        transpose(dl.data(), T, E, E, dlT.data());
        std::vector<const float*> rows(E);
        for (int e = 0; e < E; ++e) rows[e] = dlT.data() + (int64_t)e * T;
        gemm_rows(E, d, T, rows.data(), f.Xf.data(), d, dWr, d, dm->threads);
        std::vector<float> Wrf = to_f32(Wr, (int64_t)E * d);
        std::vector<const float*> drows(T);
        for (int r = 0; r < T; ++r) drows[r] = dl.data() + (int64_t)r * E;
        gemm_rows(T, d, E, drows.data(), Wrf.data(), d, dX, d, dm->threads);
    } else {
        std::fill(dX, dX + (int64_t)T * d, 0.0f);
    }

    // Experts (moe.cu:532-539, extended to up/down when h > 0).
    std::vector<float> dXg(TK * d, 0.0f);
    for (int e = 0; e < E; ++e) {
        int64_t s0 = f.offsets[e], cnt = f.offsets[e + 1] - s0;
        if (cnt == 0) {
            std::fill(dW_up[e], dW_up[e] + (int64_t)hn * d, 0.0f);
            if (h > 0) std::fill(dW_down[e], dW_down[e] + (int64_t)d * h, 0.0f);
            continue;
        }
        std::vector<float> dU;  // [cnt][hn], gradient at the first GEMM's output
        std::vector<const float*> rows(std::max<int64_t>(cnt, std::max(hn, d)));
        if (h > 0) {
            // dW_down[e] = dO^T A ; dA = dO W_down ; dU = dA * silu'(U)
            std::vector<float> dOT((int64_t)d * cnt);
            transpose(dOut.data() + s0 * d, cnt, d, d, dOT.data());
            for (int c = 0; c < d; ++c) rows[c] = dOT.data() + (int64_t)c * cnt;
            gemm_rows(d, h, (int)cnt, rows.data(), f.A.data() + s0 * h, h, dW_down[e], h, dm->threads);
            std::vector<float> Df = to_f32(W_down[e], (int64_t)d * h);
            dU.assign(cnt * h, 0.0f);
            for (int64_t m = 0; m < cnt; ++m) rows[m] = dOut.data() + (s0 + m) * d;
            gemm_rows(cnt, h, d, rows.data(), Df.data(), h, dU.data(), h, dm->threads);
            for (int64_t i = 0; i < cnt * h; ++i) dU[i] *= dsilu_f(f.U[s0 * h + i]);
        } else {
            dU.assign(dOut.begin() + s0 * d, dOut.begin() + (s0 + cnt) * d);
        }
        // dW_up[e] = dU^T Xg ; dXg = dU W_up
        std::vector<float> dUT((int64_t)hn * cnt), Xg(cnt * d);
        transpose(dU.data(), cnt, hn, hn, dUT.data());
        for (int64_t m = 0; m < cnt; ++m)
            std::memcpy(Xg.data() + m * d, f.Xf.data() + (int64_t)f.perm[s0 + m] * d, sizeof(float) * d);
        for (int n = 0; n < hn; ++n) rows[n] = dUT.data() + (int64_t)n * cnt;
        gemm_rows(hn, d, (int)cnt, rows.data(), Xg.data(), d, dW_up[e], d, dm->threads);
        std::vector<float> Uf = to_f32(W_up[e], (int64_t)hn * d);
        for (int64_t m = 0; m < cnt; ++m) rows[m] = dU.data() + m * hn;
        gemm_rows(cnt, d, hn, rows.data(), Uf.data(), d, dXg.data() + s0 * d, d, dm->threads);
    }
    // scatter_add_kernel (moe.cu:236-249): dX_r += sum_j dXg[slot(r,j)].
    run_tasks(T, dm->threads, [&](int64_t r) {
        for (int j = 0; j < K; ++j) {
            int64_t pos = f.slot_of[r * K + j];
            for (int c = 0; c < d; ++c) dX[r * d + c] += dXg[pos * d + c];
        }
    });
    return 0;
}

int orc_router_bwd(const orc_dims* dm, const float* logits, const int32_t* idx,
                   const float* s, const int32_t* counts, float aux_coef,
                   float z_coef, float* dlogits) {
    if (!dims_ok(dm) || !logits || !idx || !s || !counts || !dlogits) return -1;
    const int T = dm->T, E = dm->E;
    std::vector<float> probs((int64_t)T * E);
    for (int r = 0; r < T; ++r) {
        const float* l = logits + (int64_t)r * E;
        double mx = l[0];
        for (int e = 1; e < E; ++e) mx = std::max(mx, (double)l[e]);
        double se = 0;
        for (int e = 0; e < E; ++e) se += std::exp((double)l[e] - mx);
        for (int e = 0; e < E; ++e) probs[(int64_t)r * E + e] = (float)(std::exp((double)l[e] - mx) / se);
    }
    router_bwd_rows(T, E, dm->K, probs.data(), idx, s, nullptr, logits, counts,
                    aux_coef, z_coef, dlogits);
    return 0;
}

// ---------------------------------------------------------------------------
// fp64 twin: a second, deliberately plain implementation (no blocking, no
// canonical order) used for finite differences and to cross-check the fp32
// oracle. Same semantics as above.
int orc_loss_f64(const orc_dims* dm, const double* X, const double* Wr,
                 const double* bias, const double* W_up, const double* W_down,
                 const double* dY, double aux_coef, double z_coef,
                 double* loss, double* dX, double* dWr, double* dW_up,
                 double* dW_down, int32_t* idx_out) {
    if (!dims_ok(dm) || !X || !W_up || !dY) return -1;
    if (dm->E > 1 && !Wr) return -1;
    if (dm->h > 0 && !W_down) return -1;
    const int T = dm->T, d = dm->d, E = dm->E, K = dm->K, h = dm->h;
    const int hn = h > 0 ? h : d;
    std::vector<double> p((size_t)T * E, 1.0), lse(T, 0.0), w((size_t)T * K, 1.0);
    std::vector<int> idx((size_t)T * K, 0), cnt(E, 0);
    std::vector<double> l((size_t)T * E, 0.0);
    if (E > 1) {
        for (int r = 0; r < T; ++r) {
            for (int e = 0; e < E; ++e) {
                double v = 0;
                for (int k = 0; k < d; ++k) v += X[(size_t)r * d + k] * Wr[(size_t)e * d + k];
                l[(size_t)r * E + e] = v + (bias ? bias[e] : 0.0);
            }
            double mx = l[(size_t)r * E];
            for (int e = 1; e < E; ++e) mx = std::max(mx, l[(size_t)r * E + e]);
            double se = 0;
            for (int e = 0; e < E; ++e) se += std::exp(l[(size_t)r * E + e] - mx);
            for (int e = 0; e < E; ++e) p[(size_t)r * E + e] = std::exp(l[(size_t)r * E + e] - mx) / se;
            lse[r] = mx + std::log(se);
            std::vector<char> used(E, 0);
            double zs = 0;
            for (int j = 0; j < K; ++j) {
                int best = -1;
                double bv = 0;
                for (int e = 0; e < E; ++e)
                    if (!used[e] && (best < 0 || l[(size_t)r * E + e] > bv)) { best = e; bv = l[(size_t)r * E + e]; }
                used[best] = 1;
                idx[(size_t)r * K + j] = best;
                zs += p[(size_t)r * E + best];
            }
            for (int j = 0; j < K; ++j) w[(size_t)r * K + j] = p[(size_t)r * E + idx[(size_t)r * K + j]] / zs;
        }
    }
    for (int i = 0; i < T * K; ++i) cnt[idx[i]]++;
    if (idx_out) for (int i = 0; i < T * K; ++i) idx_out[i] = idx[i];

    // Per (r, j) expert evaluation.
    auto sig = [](double x) { return 1.0 / (1.0 + std::exp(-x)); };
    double L = 0;
    std::vector<double> s((size_t)T * K, 0.0);
    if (dX) std::fill(dX, dX + (size_t)T * d, 0.0);
    if (dWr && E > 1) std::fill(dWr, dWr + (size_t)E * d, 0.0);
    if (dW_up) std::fill(dW_up, dW_up + (size_t)E * hn * d, 0.0);
    if (dW_down && h > 0) std::fill(dW_down, dW_down + (size_t)E * d * h, 0.0);
    std::vector<double> u(hn), a(hn), o(d), du(hn), dox(d);
    for (int r = 0; r < T; ++r) {
        const double* x = X + (size_t)r * d;
        const double* dy = dY + (size_t)r * d;
        for (int j = 0; j < K; ++j) {
            int e = idx[(size_t)r * K + j];
            const double* Wu = W_up + (size_t)e * hn * d;
            for (int n = 0; n < hn; ++n) {
                double v = 0;
                for (int k = 0; k < d; ++k) v += x[k] * Wu[(size_t)n * d + k];
                u[n] = v;
                a[n] = v * sig(v);
            }
            if (h > 0) {
                const double* Wd = W_down + (size_t)e * d * h;
                for (int c = 0; c < d; ++c) {
                    double v = 0;
                    for (int n = 0; n < h; ++n) v += a[n] * Wd[(size_t)c * h + n];
                    o[c] = v;
                }
            } else {
                for (int c = 0; c < d; ++c) o[c] = a[c];
            }
            double sj = 0;
            for (int c = 0; c < d; ++c) sj += dy[c] * o[c];
            s[(size_t)r * K + j] = sj;
            double wj = w[(size_t)r * K + j];
            L += wj * sj;
            // Expert backward for this slot.
            for (int c = 0; c < d; ++c) dox[c] = wj * dy[c];
            if (h > 0) {
                const double* Wd = W_down + (size_t)e * d * h;
                for (int n = 0; n < h; ++n) {
                    double v = 0;
                    for (int c = 0; c < d; ++c) v += dox[c] * Wd[(size_t)c * h + n];
                    double sg = sig(u[n]);
                    du[n] = v * sg * (1.0 + u[n] * (1.0 - sg));
                }
                if (dW_down)
                    for (int c = 0; c < d; ++c)
                        for (int n = 0; n < h; ++n) dW_down[(size_t)e * d * h + (size_t)c * h + n] += dox[c] * a[n];
            } else {
                for (int n = 0; n < hn; ++n) {
                    double sg = sig(u[n]);
                    du[n] = dox[n] * sg * (1.0 + u[n] * (1.0 - sg));
                }
            }
            if (dW_up)
                for (int n = 0; n < hn; ++n)
                    for (int k = 0; k < d; ++k) dW_up[(size_t)e * hn * d + (size_t)n * d + k] += du[n] * x[k];
            if (dX)
                for (int n = 0; n < hn; ++n)
                    for (int k = 0; k < d; ++k) dX[(size_t)r * d + k] += du[n] * Wu[(size_t)n * d + k];
        }
    }
    if (E > 1) {
        double aux = 0, zz = 0;
        for (int e = 0; e < E; ++e) {
            double sp = 0;
            for (int r = 0; r < T; ++r) sp += p[(size_t)r * E + e];
            aux += (sp / T) * ((double)cnt[e] / ((double)T * K));
        }
        aux *= E;
        for (int r = 0; r < T; ++r) zz += lse[r] * lse[r];
        zz /= T;
        L += aux_coef * aux + z_coef * zz;
        // Router gradient: renorm + softmax + aux + z (moe.cu:199-234).
        for (int r = 0; r < T; ++r) {
            double Z = 0, sp = 0;
            for (int j = 0; j < K; ++j) {
                double pj = p[(size_t)r * E + idx[(size_t)r * K + j]];
                Z += pj;
                sp += s[(size_t)r * K + j] * pj;
            }
            std::vector<double> g(E, 0.0);
            for (int j = 0; j < K; ++j)
                g[idx[(size_t)r * K + j]] = (s[(size_t)r * K + j] * Z - sp) / (Z * Z);
            double acc = 0, expected = 0;
            for (int e = 0; e < E; ++e) {
                acc += g[e] * p[(size_t)r * E + e];
                expected += p[(size_t)r * E + e] * cnt[e] / ((double)T * K);
            }
            for (int e = 0; e < E; ++e) {
                double pe = p[(size_t)r * E + e];
                double dle = pe * (g[e] - acc) +
                             aux_coef * E / T * pe * (cnt[e] / ((double)T * K) - expected) +
                             z_coef * 2.0 / T * lse[r] * pe;
                for (int k = 0; k < d; ++k) {
                    if (dWr) dWr[(size_t)e * d + k] += dle * X[(size_t)r * d + k];
                    if (dX) dX[(size_t)r * d + k] += dle * Wr[(size_t)e * d + k];
                }
            }
        }
    }
    if (loss) *loss = L;
    return 0;
}

// ---------------------------------------------------------------------------
// MXFP4 (OCP Microscaling v1.0): blocks of 32 values share an e8m0 scale
// 2^(s-127); each value is e2m1 {0, 0.5, 1, 1.5, 2, 3, 4, 6} with a sign.
// Scale exponent = floor(log2(amax)) - 2 (the largest e2m1 exponent);
// elements are rounded to nearest, ties to the even code, and saturate at 6.
// The reference has no FP4 path; this is the build's own definition.
namespace {
const float kE2M1[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

uint8_t e2m1_encode(float v) {
    uint8_t sign = std::signbit(v) ? 8 : 0;
    float a = std::fabs(v);
    if (!(a == a)) return 0;  // NaN -> 0 (never produced from finite input)
    int best = 0;
    for (int c = 1; c < 8; ++c) {
        float dc = std::fabs(a - kE2M1[c]), db = std::fabs(a - kE2M1[best]);
        if (dc < db || (dc == db && (c % 2 == 0) && (best % 2 == 1))) best = c;
    }
    if (a >= 6.0f) best = 7;
    return (uint8_t)(sign | best);
}
}  // namespace

// LayerNorm forward (tmt-cuda/src/norm.cu:8-51): H = bf16(((x - mean) * rstd)
// * gamma + beta), each operation rounded on its own; statistics in the
// canonical order of ln_row_stats.
int orc_layernorm_fwd(int32_t T, int32_t d, const uint16_t* S, const float* gamma,
                      const float* beta, uint16_t* H, float* mean, float* rstd) {
    if (T < 0 || d <= 0 || !S || !gamma || !beta || !H || !mean || !rstd) return -1;
    for (int64_t r = 0; r < T; ++r) {
        const uint16_t* x = S + r * d;
        float m, rs;
        ln_row_stats(x, d, &m, &rs);
        mean[r] = m;
        rstd[r] = rs;
        for (int k = 0; k < d; ++k) {
            const float xm = bf(x[k]) - m;
            const float xh = xm * rs;
            const float t = xh * gamma[k];
            H[r * d + k] = tobf(t + beta[k]);
        }
    }
    return 0;
}

// LayerNorm backward (tmt-cuda/src/norm.cu:53-106) from the fp32 gradient dH
// of its output: with g = dH * gamma and xh = (x - mean) * rstd,
// dS = rstd * ((g - mean(g)) - xh * mean(g * xh)); dgamma = sum_r dH * xh,
// dbeta = sum_r dH (overwritten; ascending rows).
int orc_layernorm_bwd(int32_t T, int32_t d, const uint16_t* S, const float* dH,
                      const float* gamma, const float* mean, const float* rstd,
                      float* dS, float* dgamma, float* dbeta) {
    if (T < 0 || d <= 0 || !S || !dH || !gamma || !mean || !rstd || !dS || !dgamma || !dbeta) return -1;
    for (int k = 0; k < d; ++k) dgamma[k] = dbeta[k] = 0.0f;
    std::vector<float> xh(d), g(d);
    for (int64_t r = 0; r < T; ++r) {
        const uint16_t* x = S + r * d;
        const float* dy = dH + r * d;
        double s1 = 0.0, s2 = 0.0;
        for (int k = 0; k < d; ++k) {
            xh[k] = (bf(x[k]) - mean[r]) * rstd[r];
            g[k] = dy[k] * gamma[k];
            s1 += g[k];
            s2 += (double)g[k] * xh[k];
            dgamma[k] += dy[k] * xh[k];
            dbeta[k] += dy[k];
        }
        const float a = (float)(s1 / d), b = (float)(s2 / d);
        for (int k = 0; k < d; ++k) dS[r * d + k] = rstd[r] * ((g[k] - a) - xh[k] * b);
    }
    return 0;
}

int orc_mxfp4_quantize(const float* in, int64_t rows, int64_t n,
                       uint8_t* packed, uint8_t* scales) {
    if (!in || !packed || !scales || n % 32 != 0 || rows < 0) return -1;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < n / 32; ++b) {
            const float* v = in + r * n + b * 32;
            float amax = 0;
            for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(v[i]));
            int se = 0;  // unbiased scale exponent
            if (amax > 0) {
                int ex;
                std::frexp(amax, &ex);  // amax = f * 2^ex, f in [0.5, 1)
                se = (ex - 1) - 2;
                se = std::max(-127, std::min(127, se));
            }
            scales[r * (n / 32) + b] = (uint8_t)(se + 127);
            float inv = std::ldexp(1.0f, -se);
            for (int i = 0; i < 32; i += 2) {
                uint8_t lo = e2m1_encode(v[i] * inv), hi = e2m1_encode(v[i + 1] * inv);
                packed[r * (n / 2) + b * 16 + i / 2] = (uint8_t)(lo | (hi << 4));
            }
        }
    return 0;
}

}  // extern "C"

namespace {

constexpr int kAdamChunkElems = 8192;  // elements per chunk (one GPU workgroup)
constexpr int kAdamThreads = 256;      // threads per workgroup (4 waves of 64)

constexpr int kAdamNormThreads = 1024;  // threads of the final (one-workgroup) sum

// Fixed-order sum of nthreads per-thread values: within each wave of 64 an
// xor butterfly (offsets 32..1, every lane ends with the same value), then
// the wave sums added in order, ((w0 + w1) + w2) + ...
double adamw_block_sum(const double* t, int nthreads) {
    double tot = 0.0;
    for (int wave = 0; wave < nthreads / 64; ++wave) {
        double l[64];
        for (int i = 0; i < 64; ++i) l[i] = t[wave * 64 + i];
        for (int off = 32; off >= 1; off >>= 1) {
            double nl[64];
            for (int i = 0; i < 64; ++i) nl[i] = l[i] + l[i ^ off];
            std::memcpy(l, nl, sizeof(l));
        }
        tot = wave == 0 ? l[0] : tot + l[0];
    }
    return tot;
}

// Canonical sum of grad^2 of one chunk: thread t owns the 4-element groups
// t, t+256, t+512, ... (elements in ascending order inside a group) and
// accumulates (double)g*g from +0; then adamw_block_sum.
double adamw_chunk_sum(const float* g, int len) {
    double t[kAdamThreads];
    for (int th = 0; th < kAdamThreads; ++th) {
        double acc = 0.0;
        for (int i0 = th * 4; i0 < len; i0 += 4 * kAdamThreads)
            for (int k = 0; k < 4 && i0 + k < len; ++k) acc = acc + (double)g[i0 + k] * (double)g[i0 + k];
        t[th] = acc;
    }
    return adamw_block_sum(t, kAdamThreads);
}

uint16_t adamw_tobf(float f) {  // round to nearest even (finite values)
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffff) ? 0x40 : 0));
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

}  // namespace

extern "C" {

// The reference's per-element update (adam.cu:74-85) with the clipping scale
// of adam.cu:72-73 and the bias corrections of model.cu:721-722.
int orc_adamw_step(int32_t count, float* const* master, float* const* m, float* const* v,
                   const float* const* grad, uint16_t* const* work, const int64_t* n,
                   const int32_t* flags, float clip, float lr, float b1, float b2, float eps,
                   float wd, int32_t step, double* sumsq) {
    if (count < 0 || step < 1 || !sumsq) return -1;
    // Chunk sums in table order, then the global fixed-order sum.
    std::vector<double> part;
    for (int i = 0; i < count; ++i)
        for (int64_t s = 0; s < n[i]; s += kAdamChunkElems) {
            const int len = (int)std::min<int64_t>(kAdamChunkElems, n[i] - s);
            part.push_back((flags[i] & 1) ? adamw_chunk_sum(grad[i] + s, len) : 0.0);
        }
    double t[kAdamNormThreads];
    for (int th = 0; th < kAdamNormThreads; ++th) {
        double acc = 0.0;
        for (size_t k = th; k < part.size(); k += kAdamNormThreads) acc = acc + part[k];
        t[th] = acc;
    }
    const double s = adamw_block_sum(t, kAdamNormThreads);
    *sumsq = s;
    if (!std::isfinite(s)) return 0;  // the step is refused: nothing changes
    const float scale = clip > 0.f ? std::fmin(1.f, clip / std::fmax((float)std::sqrt(s), 1e-12f)) : 1.f;
    const float bc1 = 1.0f - powf(b1, (float)step), bc2 = 1.0f - powf(b2, (float)step);
    for (int i = 0; i < count; ++i) {
        if (!(flags[i] & 2)) continue;
        for (int64_t k = 0; k < n[i]; ++k) {
            const float g = grad[i][k] * scale;
            const float nm = b1 * m[i][k] + (1.0f - b1) * g;
            const float nv = b2 * v[i][k] + (1.0f - b2) * g * g;
            m[i][k] = nm;
            v[i][k] = nv;
            const float w = master[i][k] - lr * ((nm / bc1) / (std::sqrt(nv / bc2) + eps) + wd * master[i][k]);
            master[i][k] = w;
            if (work && work[i]) work[i][k] = adamw_tobf(w);
        }
    }
    return 0;
}

int orc_mxfp4_dequantize(const uint8_t* packed, const uint8_t* scales,
                         int64_t rows, int64_t n, float* out) {
    if (!packed || !scales || !out || n % 32 != 0 || rows < 0) return -1;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t i = 0; i < n; ++i) {
            uint8_t byte = packed[r * (n / 2) + i / 2];
            uint8_t c = (i & 1) ? (byte >> 4) : (byte & 15);
            float v = kE2M1[c & 7];
            if (c & 8) v = -v;
            int se = (int)scales[r * (n / 32) + i / 32] - 127;
            out[r * n + i] = std::ldexp(v, se);
        }
    return 0;
}

}  // extern "C"
