"""The oracle's LayerNorm (tmt-cuda/src/norm.cu:8-106 restated with a
canonical statistics order), pinned by:
  * an independent numpy restatement of that order (bit-equal H, mean, rstd);
  * fp64 LayerNorm (closed form) within bf16 rounding;
  * special cases: a constant row gives H = beta exactly; gamma scales
    around beta;
  * the backward against fp64 analytic gradients and central finite
    differences of sum(dH * LN(S)).
"""
import numpy as np

from synthetic import bf16_bits, bf16_to_f32


def _numpy_canonical(S_bits, gamma, beta):
    """Lane (k/8) mod 64 partial sums in ascending k, xor butterfly 32..1;
    every operation in float32 (x*x of a bf16 value is exact, so fmaf and
    multiply-then-add agree)."""
    T, d = S_bits.shape
    x = bf16_to_f32(S_bits)
    H = np.empty((T, d), np.uint16)
    mean = np.empty(T, np.float32)
    rstd = np.empty(T, np.float32)
    one, eps, D = np.float32(1.0), np.float32(1e-5), np.float32(d)
    for r in range(T):
        ls = np.zeros(64, np.float32)
        lq = np.zeros(64, np.float32)
        for k in range(d):
            L = (k >> 3) & 63
            v = x[r, k]
            ls[L] = np.float32(ls[L] + v)
            lq[L] = np.float32(lq[L] + np.float32(v * v))
        off = 32
        while off >= 1:
            idx = np.arange(64) ^ off
            ls = (ls + ls[idx]).astype(np.float32)
            lq = (lq + lq[idx]).astype(np.float32)
            off >>= 1
        m = np.float32(ls[0] / D)
        var = np.float32(np.float32(lq[0] / D) - np.float32(m * m))
        rs = np.float32(one / np.float32(np.sqrt(np.float32(var + eps))))
        mean[r], rstd[r] = m, rs
        xh = ((x[r] - m).astype(np.float32) * rs).astype(np.float32)
        y = ((xh * gamma).astype(np.float32) + beta).astype(np.float32)
        H[r] = bf16_bits(y)
    return H, mean, rstd


def _case(T, d, seed):
    rng = np.random.default_rng(seed)
    S = bf16_bits((rng.standard_normal((T, d)) * 1.7 + 0.3).astype(np.float32))
    gamma = (1.0 + 0.2 * rng.standard_normal(d)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(d)).astype(np.float32)
    return S, gamma, beta


def test_layernorm_canonical_order_is_pinned(orc):
    for T, d in ((5, 256), (3, 1088), (2, 64)):
        S, g, b = _case(T, d, T + d)
        ref = orc.layernorm(S, g, b)
        H, mean, rstd = _numpy_canonical(S, g, b)
        assert np.array_equal(ref["mean"].view(np.uint32), mean.view(np.uint32))
        assert np.array_equal(ref["rstd"].view(np.uint32), rstd.view(np.uint32))
        assert np.array_equal(ref["H"], H)


def test_layernorm_matches_fp64(orc):
    S, g, b = _case(64, 1024, 3)
    ref = orc.layernorm(S, g, b)
    x = bf16_to_f32(S).astype(np.float64)
    m = x.mean(1, keepdims=True)
    v = x.var(1, keepdims=True)
    y = (x - m) / np.sqrt(v + 1e-5) * g + b
    h = bf16_to_f32(ref["H"]).astype(np.float64)
    assert np.all(np.abs(h - y) <= 2.0 ** -8 * np.abs(y) + 1e-6)
    assert np.allclose(ref["mean"], m[:, 0], rtol=1e-6, atol=1e-6)
    assert np.allclose(ref["rstd"], 1 / np.sqrt(v[:, 0] + 1e-5), rtol=1e-5)


def test_layernorm_special_cases(orc):
    d = 128
    S = np.full((2, d), bf16_bits(np.array([1.5], np.float32))[0], np.uint16)
    g = np.linspace(0.5, 2.0, d).astype(np.float32)
    b = np.linspace(-1.0, 1.0, d).astype(np.float32)
    ref = orc.layernorm(S, g, b)
    assert np.array_equal(ref["H"], np.tile(bf16_bits(b), (2, 1)))   # constant row -> beta
    assert np.all(ref["mean"] == np.float32(1.5))
    assert np.allclose(ref["rstd"], 1 / np.sqrt(np.float32(1e-5)), rtol=1e-6)
    # gamma doubles the centred part, beta shifts it
    S2, _, _ = _case(3, d, 9)
    one = np.ones(d, np.float32)
    zero = np.zeros(d, np.float32)
    h1 = bf16_to_f32(orc.layernorm(S2, one, zero)["H"])
    h2 = bf16_to_f32(orc.layernorm(S2, 2 * one, one)["H"])
    assert np.allclose(h2, 2 * h1 + 1, rtol=2.0 ** -7, atol=2.0 ** -6)


def _ln64(x, g, b):
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + 1e-5) * g + b


def test_layernorm_backward(orc):
    T, d = 6, 128
    S, g, b = _case(T, d, 21)
    fwd = orc.layernorm(S, g, b)
    rng = np.random.default_rng(5)
    dH = rng.standard_normal((T, d)).astype(np.float32)
    got = orc.layernorm_bwd(S, dH, g, fwd["mean"], fwd["rstd"])
    x = bf16_to_f32(S).astype(np.float64)
    m = x.mean(1, keepdims=True)
    rs = 1 / np.sqrt(((x - m) ** 2).mean(1, keepdims=True) + 1e-5)
    xh = (x - m) * rs
    gg = dH.astype(np.float64) * g
    dS = rs * (gg - gg.mean(1, keepdims=True) - xh * (gg * xh).mean(1, keepdims=True))
    assert np.allclose(got["dS"], dS, rtol=1e-4, atol=1e-5)
    assert np.allclose(got["dgamma"], (dH * xh).sum(0), rtol=1e-4, atol=1e-4)
    assert np.allclose(got["dbeta"], dH.sum(0), rtol=1e-5, atol=1e-5)
    # central differences of sum(dH * LN(S)) on a few elements
    loss = lambda xx: float((dH.astype(np.float64) * _ln64(xx, g, b)).sum())
    for (r, k) in ((0, 0), (2, 17), (5, 127), (3, 64)):
        eps = 1e-4
        xp, xm = x.copy(), x.copy()
        xp[r, k] += eps
        xm[r, k] -= eps
        fd = (loss(xp) - loss(xm)) / (2 * eps)
        assert abs(fd - got["dS"][r, k]) <= 1e-3 * max(1.0, abs(fd)), (r, k, fd, got["dS"][r, k])
