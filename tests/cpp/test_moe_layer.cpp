// test_moe_layer.cpp -- the reference's MoE layer tests, restated against the
// C++ operator interface of include/tmt_moe.hpp (moe_keep_alloc /
// moe_forward / moe_aux_from / moe_backward), in the reference's own style:
// a PASS line per test, a message and exit(1) on the first failure.
//
//   test_router        tmt-cuda/src/architecture_test.cu:62-87
//   test_moe_backward  tmt-cuda/src/architecture_test.cu:228-264
//   experts limit      tmt-cuda/tests/cli.sh:30-32 (the limit here is 64)
//   test_layernorm     layernorm_fwd / layernorm_bwd (norm.cu:96-106) against fp64
//   test_model_flow    the model's multi-layer use: model.cu:252-258, 512-514,
//                      542-549, 672-677; capi.cu:131-136; train_main.cu:232-248
//
// Usage: test_moe_layer            all GPU tests
//        test_moe_layer reject     only the configuration check (no GPU use)
#include "tmt_moe.hpp"

#include <cmath>
#include <cstring>
#include <random>
#include <string>
#include <vector>

static void require(bool ok, const char* what) {
    if (!ok) {
        std::printf("FAIL %s\n", what);
        std::exit(1);
    }
}
static void near(double got, double want, double atol, double rtol, const char* what) {
    if (!(std::fabs(got - want) <= atol + rtol * std::fabs(want))) {
        std::printf("FAIL %s: got %.9g want %.9g\n", what, got, want);
        std::exit(1);
    }
}
static double rel_l2(const std::vector<float>& x, const std::vector<float>& y) {
    double e = 0, n = 0;
    for (size_t i = 0; i < x.size(); ++i) {
        e += (double(x[i]) - y[i]) * (double(x[i]) - y[i]);
        n += double(y[i]) * y[i];
    }
    return n > 0 ? std::sqrt(e / n) : std::sqrt(e);
}

// bf16 as uint16 bit patterns, round to nearest even.
static uint16_t f2bf(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
static float bf2f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

struct Device {  // device allocations of one test, freed at scope end
    std::vector<void*> ptrs;
    ~Device() {
        for (void* p : ptrs) (void)hipFree(p);
    }
    template <class T>
    T* alloc(size_t n) {
        void* p = nullptr;
        tmt_moe_detail::check_hip(hipMalloc(&p, n * sizeof(T) + 16), "hipMalloc");
        tmt_moe_detail::check_hip(hipMemset(p, 0, n * sizeof(T) + 16), "hipMemset");
        ptrs.push_back(p);
        return (T*)p;
    }
    template <class T>
    T* upload(const std::vector<T>& v) {
        T* p = alloc<T>(v.size());
        tmt_moe_detail::check_hip(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice), "upload");
        return p;
    }
};
template <class T>
static std::vector<T> download(const T* p, size_t n) {
    std::vector<T> v(n);
    tmt_moe_detail::check_hip(hipDeviceSynchronize(), "sync");
    tmt_moe_detail::check_hip(hipMemcpy(v.data(), p, n * sizeof(T), hipMemcpyDeviceToHost), "download");
    return v;
}
static std::vector<float> to_f32(const std::vector<uint16_t>& b) {
    std::vector<float> f(b.size());
    for (size_t i = 0; i < b.size(); ++i) f[i] = bf2f(b[i]);
    return f;
}
static std::vector<uint16_t> normal_bf16(std::mt19937& g, size_t n, float std) {
    std::normal_distribution<float> nd(0.f, std);
    std::vector<uint16_t> v(n);
    for (auto& x : v) x = f2bf(nd(g));
    return v;
}
static std::vector<uint16_t> uniform_bf16(std::mt19937& g, size_t n, float a) {
    std::uniform_real_distribution<float> ud(-a, a);
    std::vector<uint16_t> v(n);
    for (auto& x : v) x = f2bf(ud(g));
    return v;
}

// Router regulariser gradient against central differences of the aux and
// z-loss objective on the layer's own logits (as test_router), with zero
// upstream gradient so only the regulariser reaches the router; checked
// through dWrouter = dlogits^T X and the router part of dX = dlogits Wr.
static void test_router() {
    constexpr int N = 5, E = 4, K = 2, D = 16;  // small_config's dim (architecture_test.cu:88-89)
    std::mt19937 g(1234);
    auto X = normal_bf16(g, (size_t)N * D, 1.f), Wr = normal_bf16(g, (size_t)E * D, 0.125f);
    std::vector<std::vector<uint16_t>> We(E);
    for (auto& w : We) w = uniform_bf16(g, (size_t)D * D, std::sqrt(1.f / D));
    Device dev;
    uint16_t *dXd = dev.upload(X), *dWr = dev.upload(Wr), *Y = dev.alloc<uint16_t>((size_t)N * D);
    uint16_t* dY = dev.alloc<uint16_t>((size_t)N * D);
    uint16_t* dXo = dev.alloc<uint16_t>((size_t)N * D);
    float* dWrouter = dev.alloc<float>((size_t)E * D);
    std::vector<uint16_t*> Wx(E);
    std::vector<float*> dWx(E);
    for (int e = 0; e < E; ++e) {
        Wx[e] = dev.upload(We[e]);
        dWx[e] = dev.alloc<float>((size_t)D * D);
    }
    MoeKeep k;
    MoeWs w;
    moe_keep_alloc(k, N, E, K, D);
    moe_ws_alloc(w, N, E, K, D);
    for (auto coef : {std::pair<float, float>{.7f, 0.f}, {0.f, .3f}}) {
        moe_forward(dXd, dWr, Wx.data(), Y, k, w, N, E, K, D, 0.f);
        moe_backward(dY, Wx.data(), dWr, dWrouter, dWx.data(), dXo, k, w, coef.first, coef.second);
        std::vector<float> logits((size_t)N * E);
        tmt_moe_detail::check(tmt_moe_read_routing(k.handle, k.stream, logits.data(), nullptr, nullptr,
                                                   nullptr, nullptr, nullptr, nullptr), "read_routing");
        const int32_t* cnt = k.hcnt;
        auto objective = [&](const std::vector<double>& z) {
            double loss = 0;
            for (int r = 0; r < N; ++r) {
                double sum = 0;
                for (int e = 0; e < E; ++e) sum += std::exp(z[r * E + e]);
                double lse = std::log(sum);
                loss += coef.second * lse * lse / N;
                for (int e = 0; e < E; ++e)
                    loss += coef.first * E / N * std::exp(z[r * E + e]) / sum * cnt[e] / (N * K);
            }
            return loss;
        };
        std::vector<double> z(logits.begin(), logits.end()), dl((size_t)N * E);
        for (int i = 0; i < N * E; ++i) {
            double old = z[i], eps = 1e-4;
            z[i] = old + eps;
            double hi = objective(z);
            z[i] = old - eps;
            double lo = objective(z);
            z[i] = old;
            dl[i] = (hi - lo) / (2 * eps);
        }
        auto gWr = download(dWrouter, (size_t)E * D);
        auto gX = to_f32(download(dXo, (size_t)N * D));
        for (int e = 0; e < E; ++e)
            for (int c = 0; c < D; ++c) {
                double want = 0;
                for (int r = 0; r < N; ++r) want += dl[r * E + e] * bf2f(X[(size_t)r * D + c]);
                near(gWr[(size_t)e * D + c], want, 2e-5, 2e-3, "router regularizer gradient (dWrouter)");
            }
        for (int r = 0; r < N; ++r)
            for (int c = 0; c < D; ++c) {
                double want = 0;
                for (int e = 0; e < E; ++e) want += dl[r * E + e] * bf2f(Wr[(size_t)e * D + c]);
                near(gX[(size_t)r * D + c], want, 1e-5, 1e-2, "router regularizer gradient (dX)");
            }
        for (int e = 0; e < E; ++e) {
            auto gw = download(dWx[e], (size_t)D * D);
            for (float v : gw) require(v == 0.f, "expert gradient without upstream gradient is not zero");
        }
    }
    moe_keep_free(k);
    moe_ws_free(w);
    std::puts("PASS MoE auxiliary and z-loss finite-difference gradients");
}

// Two experts with identical weights, both selected (renormalised weights sum
// to 1), compute exactly the dense layer: forward, summed expert gradients
// and the input gradient must match the E=1 path (as test_moe_backward, which
// runs small_config: dim 16, batch 2 x seqlen 7, architecture_test.cu:88-89).
static void identical_experts(int D, int hidden) {
    constexpr int N = 14;  // batch 2 x seqlen 7
    const int hn = hidden > 0 ? hidden : D;
    std::mt19937 g(99 + hidden + D);
    auto X = normal_bf16(g, (size_t)N * D, 1.f), Y0 = normal_bf16(g, (size_t)N * D, 1.f);
    auto dYh = normal_bf16(g, (size_t)N * D, 1.f), Wr = normal_bf16(g, (size_t)2 * D, 0.02f);
    auto Wu = uniform_bf16(g, (size_t)hn * D, std::sqrt(1.f / D));
    auto Wd = hidden > 0 ? uniform_bf16(g, (size_t)D * hidden, std::sqrt(1.f / hidden)) : std::vector<uint16_t>();
    Device dev;
    uint16_t *dXd = dev.upload(X), *dWr = dev.upload(Wr), *dY = dev.upload(dYh);
    uint16_t *Wu1 = dev.upload(Wu), *Wu2 = dev.upload(Wu);
    uint16_t *Wd1 = hidden > 0 ? dev.upload(Wd) : nullptr, *Wd2 = hidden > 0 ? dev.upload(Wd) : nullptr;
    std::vector<float> y[2], dx[2], dwu[2], dwd[2];
    for (int moe = 0; moe < 2; ++moe) {
        const int E = moe ? 2 : 1, K = E;
        uint16_t* Y = dev.upload(Y0);
        uint16_t* dX = dev.alloc<uint16_t>((size_t)N * D);
        float* dWrouter = dev.alloc<float>((size_t)E * D);
        uint16_t* Wup[2] = {Wu1, Wu2};
        uint16_t* Wdn[2] = {Wd1, Wd2};
        float* dWup[2] = {dev.alloc<float>((size_t)hn * D), dev.alloc<float>((size_t)hn * D)};
        float* dWdn[2] = {hidden > 0 ? dev.alloc<float>((size_t)D * hidden) : nullptr,
                          hidden > 0 ? dev.alloc<float>((size_t)D * hidden) : nullptr};
        MoeKeep k;
        MoeWs w;
        moe_keep_alloc(k, N, E, K, D, hidden);
        float aux;
        if (hidden > 0) {
            aux = moe_forward(dXd, dWr, Wup, Wdn, Y, k, w, N, E, K, D, 1.0f);
            moe_backward(dY, Wup, Wdn, dWr, dWrouter, dWup, dWdn, dX, k, w, 0.f, 0.f);
        } else {
            aux = moe_forward(dXd, dWr, Wup, Y, k, w, N, E, K, D, 1.0f);
            moe_backward(dY, Wup, dWr, dWrouter, dWup, dX, k, w, 0.f, 0.f);
        }
        if (E == 2) near(aux, 1.0, 1e-6, 1e-6, "aux with both experts always selected is not 1");
        y[moe] = to_f32(download(Y, (size_t)N * D));
        dx[moe] = to_f32(download(dX, (size_t)N * D));
        dwu[moe] = download(dWup[0], (size_t)hn * D);
        if (hidden > 0) dwd[moe] = download(dWdn[0], (size_t)D * hidden);
        if (E == 2) {
            auto b = download(dWup[1], (size_t)hn * D);
            for (size_t i = 0; i < b.size(); ++i) dwu[moe][i] += b[i];
            if (hidden > 0) {
                auto c = download(dWdn[1], (size_t)D * hidden);
                for (size_t i = 0; i < c.size(); ++i) dwd[moe][i] += c[i];
            }
            auto gr = download(dWrouter, (size_t)E * D);
            double mx = 0;
            for (float v : gr) mx = std::fmax(mx, std::fabs(v));
            near(mx, 0, 1e-4, 0, "router gradient of identical experts is not zero");
        }
        moe_keep_free(k);
    }
    near(rel_l2(y[1], y[0]), 0, 5e-3, 0, "MoE with identical experts differs from dense forward");
    near(rel_l2(dwu[1], dwu[0]), 0, 0.03, 0, "summed MoE expert gradients differ from dense");
    if (hidden > 0) near(rel_l2(dwd[1], dwd[0]), 0, 0.03, 0, "summed MoE down-projection gradients differ from dense");
    near(rel_l2(dx[1], dx[0]), 0, 0.03, 0, "input gradient through MoE differs from dense");
}
static void test_moe_backward() {
    identical_experts(16, 0);
    std::puts("PASS MoE backward: identical experts reproduce dense expert and input gradients (dim 16)");
    identical_experts(64, 0);
    std::puts("PASS MoE backward: identical experts reproduce dense expert and input gradients (dim 64)");
    identical_experts(16, 40);
    std::puts("PASS MoE backward (up/SiLU/down experts, dim 16, hidden 40): identical experts reproduce the dense layer");
    identical_experts(64, 128);
    std::puts("PASS MoE backward (up/SiLU/down experts): identical experts reproduce the dense layer");
}

// Deferred statistics (MoeKeep::stat, model.cu:255-258, 542-549) give the
// same aux and z-loss as the immediate read, and counts that sum to N*K.
static void test_deferred_stats() {
    constexpr int N = 200, E = 8, K = 2, D = 128;
    std::mt19937 g(7);
    auto X = normal_bf16(g, (size_t)N * D, 1.f), Wr = normal_bf16(g, (size_t)E * D, 0.1f);
    Device dev;
    uint16_t *dXd = dev.upload(X), *dWr = dev.upload(Wr), *Y = dev.alloc<uint16_t>((size_t)N * D);
    std::vector<uint16_t*> Wx(E);
    for (int e = 0; e < E; ++e) Wx[e] = dev.upload(uniform_bf16(g, (size_t)D * D, std::sqrt(1.f / D)));
    float* slot = dev.alloc<float>(E + 1);
    MoeKeep k;
    MoeWs w;
    moe_keep_alloc(k, N, E, K, D);
    float aux_now = moe_forward(dXd, dWr, Wx.data(), Y, k, w, N, E, K, D, 0.f);
    float z_now = k.zloss;
    k.stat = slot;
    float r = moe_forward(dXd, dWr, Wx.data(), Y, k, w, N, E, K, D, 0.f);
    require(r == 0.f && k.zloss == 0.f, "deferred moe_forward must return 0 and leave zloss 0");
    std::memset(k.hcnt, 0, sizeof(k.hcnt));
    auto hs = download(slot, E + 1);
    float aux_late = moe_aux_from(k, hs.data());
    require(aux_late == aux_now, "deferred aux differs from the immediate value");
    require(k.zloss == z_now, "deferred z-loss differs from the immediate value");
    long total = 0;
    for (int e = 0; e < E; ++e) total += k.hcnt[e];
    require(total == (long)N * K, "expert counts do not sum to N*K");
    moe_keep_free(k);
    std::puts("PASS deferred router statistics equal the immediate read");
}

// The recurrent model's use of the layer (model.cu:252-258, 512-514,
// 542-549, 672-677; capi.cu:131-136; train_main.cu:232-248): three layers
// with E = 32 (above the reference's old limit of 16), one shared MoeWs
// (checked bit for bit against private workspaces),
// residual add through beta = 1, statistics deferred into per-layer slots
// with a stride of 17 floats and read with one copy, expert counts, the
// router balance line, and the backward in reverse layer order with the
// coefficients divided by L.
static void test_model_flow() {
    constexpr int L = 3, N = 96, E = 32, K = 4, D = 64;
    const float aux_c = 0.1f, z_c = 1e-3f;
    std::mt19937 g(11);
    Device dev;
    MoeWs ws;
    moe_ws_alloc(ws, N, E, K, D);
    std::vector<MoeKeep> layers(L), immediate(L);
    std::vector<uint16_t*> Wr(L);
    std::vector<std::vector<uint16_t*>> Wx(L, std::vector<uint16_t*>(E));
    std::vector<std::vector<float*>> dWx(L, std::vector<float*>(E));
    std::vector<float*> dWr(L);
    float* stats = dev.alloc<float>((size_t)L * 17);
    for (int l = 0; l < L; ++l) {
        Wr[l] = dev.upload(normal_bf16(g, (size_t)E * D, 0.2f));
        for (int e = 0; e < E; ++e) {
            Wx[l][e] = dev.upload(uniform_bf16(g, (size_t)D * D, std::sqrt(1.f / D)));
            dWx[l][e] = dev.alloc<float>((size_t)D * D);
        }
        dWr[l] = dev.alloc<float>((size_t)E * D);
        moe_keep_alloc(layers[l], N, E, K, D);
        moe_keep_alloc(immediate[l], N, E, K, D);
        layers[l].stat = stats + (size_t)l * 17;
    }
    // forward: X_{l+1} = X_l + MoE_l(X_l)
    std::vector<uint16_t*> X(L + 1);
    X[0] = dev.upload(normal_bf16(g, (size_t)N * D, 1.f));
    for (int l = 0; l < L; ++l) {
        X[l + 1] = dev.alloc<uint16_t>((size_t)N * D);
        tmt_moe_detail::check_hip(hipMemcpy(X[l + 1], X[l], (size_t)N * D * 2, hipMemcpyDeviceToDevice), "copy");
        const float r = moe_forward(X[l], Wr[l], Wx[l].data(), X[l + 1], layers[l], ws, N, E, K, D, 1.0f);
        require(r == 0.f, "deferred moe_forward returns 0");
    }
    auto hs = download(stats, (size_t)L * 17);  // the one host read of the step
    float aux_acc = 0, z_acc = 0;
    for (int l = 0; l < L; ++l) {
        aux_acc += moe_aux_from(layers[l], &hs[(size_t)l * 17]);
        z_acc += layers[l].zloss;
        // the same layer read immediately gives the same statistics; these
        // copies run on private workspaces (an MoeWs that was never allocated)
        uint16_t* Yi = dev.alloc<uint16_t>((size_t)N * D);
        MoeWs priv;
        const float ai = moe_forward(X[l], Wr[l], Wx[l].data(), Yi, immediate[l], priv, N, E, K, D, 0.f);
        require(ai == hs[(size_t)l * 17] && immediate[l].zloss == layers[l].zloss,
                "deferred statistics differ from the immediate read");
    }
    require(std::isfinite(aux_acc) && std::isfinite(z_acc) && aux_acc > 0.f, "accumulated aux / z");
    // expert counts (tmt_model_expert_counts) and the router balance line
    std::vector<int64_t> counts((size_t)L * E);
    moe_expert_counts(layers.data(), L, counts.data());
    int zeros = 0;
    for (int l = 0; l < L; ++l) {
        int64_t tot = 0;
        for (int e = 0; e < E; ++e) {
            tot += counts[(size_t)l * E + e];
            zeros += counts[(size_t)l * E + e] == 0;
        }
        require(tot == (int64_t)N * K, "expert counts of a layer do not sum to N*K");
    }
    const MoeBalance b = moe_router_balance(counts.data(), L, E);
    require(b.pairs == L * E && b.min <= 1.0 && b.max >= 1.0, "balance shares around 1");
    require(b.dead == zeros, "dead experts are the ones with no tokens (mean count 12, threshold 0.12)");
    std::vector<int64_t> flat((size_t)L * E, 5);
    MoeBalance u = moe_router_balance(flat.data(), L, E);
    require(u.min == 1.0 && u.max == 1.0 && u.dead == 0, "uniform counts give shares of exactly 1");
    flat[7] = 0;
    u = moe_router_balance(flat.data(), L, E);
    require(u.min == 0.0 && u.dead == 1, "a silent expert is dead");
    // backward, last layer first, coefficients / L
    uint16_t* dY = dev.upload(normal_bf16(g, (size_t)N * D, 1.f));
    uint16_t* dXl = dev.alloc<uint16_t>((size_t)N * D);
    uint16_t* dXp = dev.alloc<uint16_t>((size_t)N * D);
    float* dWrp = dev.alloc<float>((size_t)E * D);
    std::vector<float*> dWxp(E);
    for (int e = 0; e < E; ++e) dWxp[e] = dev.alloc<float>((size_t)D * D);
    for (int l = L - 1; l >= 0; --l) {
        moe_backward(dY, Wx[l].data(), Wr[l], dWr[l], dWx[l].data(), dXl, layers[l], ws, aux_c / L, z_c / L);
        // the same backward on the layer copy with a private workspace: the
        // shared workspace gives the same bits
        MoeWs priv;
        moe_backward(dY, Wx[l].data(), Wr[l], dWrp, dWxp.data(), dXp, immediate[l], priv, aux_c / L, z_c / L);
        require(download(dXl, (size_t)N * D) == download(dXp, (size_t)N * D) &&
                    download(dWr[l], (size_t)E * D) == download(dWrp, (size_t)E * D) &&
                    download(dWx[l][E - 1], (size_t)D * D) == download(dWxp[E - 1], (size_t)D * D),
                "backward over the shared workspace differs from a private workspace");
        auto gx = to_f32(download(dXl, (size_t)N * D));
        auto gr = download(dWr[l], (size_t)E * D);
        for (float v : gx) require(std::isfinite(v), "dX finite");
        double nr = 0;
        for (float v : gr) nr += (double)v * v;
        require(nr > 0 && std::isfinite(nr), "router gradient written");
    }
    for (int l = 0; l < L; ++l) {
        moe_keep_free(layers[l]);
        moe_keep_free(immediate[l]);
    }
    moe_ws_free(ws);
    std::printf("PASS model flow: %d layers, E=%d, deferred statistics, counts, balance min %.3f max %.3f dead %ld/%d\n",
                L, E, b.min, b.max, b.dead, b.pairs);
}

// layernorm_fwd / layernorm_bwd (norm.cu:96-106) against an fp64 host
// LayerNorm on the same bf16 inputs, and the fused moe path's input side:
// rows with offsets and scales, ragged D.
static void test_layernorm() {
    const int N = 77, D = 320;
    std::mt19937 g(21);
    std::normal_distribution<float> nd(0.f, 1.f);
    std::vector<uint16_t> X(N * D), dY(N * D);
    std::vector<float> gamma(D), beta(D);
    for (int r = 0; r < N; ++r) {
        const float sc = std::exp(nd(g)), sh = nd(g);
        for (int k = 0; k < D; ++k) X[r * D + k] = f2bf(nd(g) * sc + sh);
    }
    for (auto& v : dY) v = f2bf(nd(g));
    for (int k = 0; k < D; ++k) {
        gamma[k] = 1.f + 0.2f * nd(g);
        beta[k] = 0.1f * nd(g);
    }
    Device dv;
    const uint16_t* dX_in = dv.upload(X);
    const uint16_t* ddY = dv.upload(dY);
    const float* dg = dv.upload(gamma);
    const float* db = dv.upload(beta);
    uint16_t* dYout = dv.alloc<uint16_t>(N * D);
    uint16_t* dXout = dv.alloc<uint16_t>(N * D);
    float* mean = dv.alloc<float>(N);
    float* rstd = dv.alloc<float>(N);
    float* dG = dv.alloc<float>(D);
    float* dB = dv.alloc<float>(D);
    layernorm_fwd(dX_in, dg, db, dYout, mean, rstd, N, D);
    layernorm_bwd(dX_in, ddY, dg, mean, rstd, dXout, dG, dB, N, D);
    const auto H = to_f32(download(dYout, N * D));
    const auto dXg = to_f32(download(dXout, N * D));
    const auto dGg = download(dG, D), dBg = download(dB, D);
    std::vector<float> Href(N * D), dXref(N * D), dGref(D, 0.f), dBref(D, 0.f);
    std::vector<double> acc_g(D, 0.0), acc_b(D, 0.0);
    for (int r = 0; r < N; ++r) {
        double s = 0, q = 0;
        for (int k = 0; k < D; ++k) s += bf2f(X[r * D + k]);
        const double m = s / D;
        for (int k = 0; k < D; ++k) q += (bf2f(X[r * D + k]) - m) * (bf2f(X[r * D + k]) - m);
        const double rs = 1.0 / std::sqrt(q / D + 1e-5);
        double s1 = 0, s2 = 0;
        for (int k = 0; k < D; ++k) {
            const double xh = (bf2f(X[r * D + k]) - m) * rs, gy = bf2f(dY[r * D + k]) * gamma[k];
            Href[r * D + k] = (float)(xh * gamma[k] + beta[k]);
            s1 += gy;
            s2 += gy * xh;
            acc_g[k] += bf2f(dY[r * D + k]) * xh;
            acc_b[k] += bf2f(dY[r * D + k]);
        }
        for (int k = 0; k < D; ++k) {
            const double xh = (bf2f(X[r * D + k]) - m) * rs, gy = bf2f(dY[r * D + k]) * gamma[k];
            dXref[r * D + k] = (float)(rs * (gy - s1 / D - xh * s2 / D));
        }
    }
    for (int k = 0; k < D; ++k) {
        dGref[k] = (float)acc_g[k];
        dBref[k] = (float)acc_b[k];
    }
    require(rel_l2(H, Href) < 5e-3, "layernorm_fwd output");
    require(rel_l2(dXg, dXref) < 1e-2, "layernorm_bwd dX");
    require(rel_l2(dGg, dGref) < 1e-3, "layernorm_bwd dGamma");
    require(rel_l2(dBg, dBref) < 1e-5, "layernorm_bwd dBeta");
    std::puts("PASS layernorm_fwd / layernorm_bwd match an fp64 LayerNorm");
}

int main(int argc, char** argv) {
    if (argc > 1 && std::string(argv[1]) == "reject") {
        MoeKeep k;
        moe_keep_alloc(k, 8, 65, 2, 64);  // exits(1): more than 64 experts
        std::puts("FAIL experts=65 was accepted");
        return 2;
    }
    test_router();
    test_moe_backward();
    test_deferred_stats();
    test_layernorm();
    test_model_flow();
    std::puts("ALL PASS");
    return 0;
}
