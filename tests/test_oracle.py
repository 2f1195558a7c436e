"""Pins the CPU oracle (oracle/moe_oracle.cpp) before it is trusted.

The reference ships no golden files (its MoE tests build inputs from
formulas, tmt-cuda/src/architecture_test.cu:62-87, 231-264), so each oracle
function is pinned here by one of: a restated reference known-answer test,
finite differences of an independent fp64 implementation, closed forms and
special cases, brute force, or the committed torch-autograd fixture.
"""
import math
import os

import numpy as np
import pytest

from synthetic import bf16_bits, bf16_to_f32

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def near(got, ref, atol, rtol, what):
    # architecture_test.cu:18-23
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    bad = ~(np.abs(got - ref) <= atol + rtol * np.abs(ref))
    assert not bad.any(), f"{what}: got {got[bad][:5]} expected {ref[bad][:5]}"


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def topk_stable(logits, K):
    """Independent top-k: stable sort on -logit (ties -> lower index)."""
    return np.argsort(-np.asarray(logits, np.float64), axis=1, kind="stable")[:, :K].astype(np.int32)


# ---------------------------------------------------------------- router --

def test_router_regularizer_gradient_fd(orc):
    """Restates test_router (architecture_test.cu:62-87): N=5, E=4, K=2,
    logits = 2 sin(0.43 i), s = 0, (aux, z) in {(0.7, 0), (0, 0.3)}; the
    analytic router gradient must match central differences (eps 1e-4)
    within atol 2e-6 / rtol 2e-4."""
    N, E, K = 5, 4, 2
    logits = (np.sin(np.arange(N * E, dtype=np.float32) * np.float32(0.43)) * 2).astype(np.float32)
    logits = logits.reshape(N, E)
    idx = topk_stable(logits, K)
    cnt = np.bincount(idx.ravel(), minlength=E)
    s = np.zeros((N, K), np.float32)
    for aux, zc in ((0.7, 0.0), (0.0, 0.3)):
        got = orc.router_bwd(logits, idx, s, cnt, aux, zc)

        def objective(z):
            z = z.reshape(N, E)
            loss = 0.0
            for r in range(N):
                ex = np.exp(z[r])
                ssum = ex.sum()
                lse = math.log(ssum)
                loss += zc * lse * lse / N
                loss += (aux * E / N * ex / ssum * cnt / (N * K)).sum()
            return loss

        z0 = logits.astype(np.float64).ravel()
        for i in range(N * E):
            zp, zm = z0.copy(), z0.copy()
            zp[i] += 1e-4
            zm[i] -= 1e-4
            fd = (objective(zp) - objective(zm)) / 2e-4
            near(got.ravel()[i], fd, 2e-6, 2e-4, "router regularizer gradient")


def _canonical_f32(x, w):
    """Independent numpy restatement of the canonical order, valid when every
    product x_k*w_k is exact in fp32 (then fmaf == one fp32 addition)."""
    d = x.size
    prod = (x.astype(np.float64) * w.astype(np.float64)).astype(np.float32)
    assert np.all(prod.astype(np.float64) == x.astype(np.float64) * w.astype(np.float64))
    lane = np.zeros(64, np.float32)
    for k in range(d):
        L = (k // 8) % 64
        lane[L] = np.float32(lane[L] + prod[k])
    for off in (32, 16, 8, 4, 2, 1):
        lane = (lane + lane[np.arange(64) ^ off]).astype(np.float32)
    return lane[0], prod


@pytest.mark.parametrize("d", [256, 1024, 1536])
def test_canonical_logit_order_is_pinned(orc, d):
    """Products are exact (4-bit mantissas, wide exponents) so the sum is
    order-sensitive; the oracle must equal the documented lane/butterfly
    order bit for bit and differ from a plain sequential sum."""
    rng = np.random.default_rng(d)
    m1 = rng.integers(1, 16, d) * rng.choice([-1, 1], d)
    m2 = rng.integers(1, 16, d) * rng.choice([-1, 1], d)
    x = (m1 * np.exp2(rng.integers(-12, 12, d))).astype(np.float32)
    w = (m2 * np.exp2(rng.integers(-12, 12, d))).astype(np.float32)
    xb, wb = bf16_bits(x), bf16_bits(w)
    assert np.all(bf16_to_f32(xb) == x) and np.all(bf16_to_f32(wb) == w)
    want, prod = _canonical_f32(x, w)
    got = orc.router_logit(xb, wb)
    assert np.float32(got).view(np.uint32) == want.view(np.uint32)
    seq = np.float32(0)
    for p in prod:
        seq = np.float32(seq + p)
    assert seq != want, "inputs must make the summation order observable"


def test_canonical_logit_accuracy(orc):
    rng = np.random.default_rng(7)
    for d in (128, 512, 1024):
        x = bf16_bits(rng.standard_normal(d).astype(np.float32))
        w = bf16_bits((rng.standard_normal(d) / math.sqrt(d)).astype(np.float32))
        ref = float(np.dot(bf16_to_f32(x).astype(np.float64), bf16_to_f32(w).astype(np.float64)))
        bound = d * 2.0 ** -23 * float(np.sum(np.abs(bf16_to_f32(x) * bf16_to_f32(w))))
        assert abs(orc.router_logit(x, w) - ref) <= bound


def test_router_against_independent_numpy(orc):
    rng = np.random.default_rng(11)
    T, d, E, K = 300, 256, 8, 3
    X = bf16_bits(rng.standard_normal((T, d)).astype(np.float32))
    Wr = bf16_bits((rng.standard_normal((E, d)) / 16).astype(np.float32))
    bias = rng.standard_normal(E).astype(np.float32)
    out = orc.router(X, Wr, K, bias=bias)
    for r in range(0, T, 37):
        for e in range(E):
            v = np.float32(orc.router_logit(X[r], Wr[e])) + bias[e]
            assert np.float32(v).view(np.uint32) == out["logits"][r, e].view(np.uint32)
    L = out["logits"].astype(np.float64)
    P = np.exp(L - L.max(1, keepdims=True))
    P /= P.sum(1, keepdims=True)
    near(out["probs"], P, 1e-7, 1e-6, "softmax")
    idx = topk_stable(L, K)
    assert np.array_equal(out["idx"], idx)
    psel = np.take_along_axis(out["probs"].astype(np.float64), idx, 1)
    near(out["gate"], psel / psel.sum(1, keepdims=True), 1e-7, 1e-6, "renormalised gate")
    lse = L.max(1) + np.log(np.exp(L - L.max(1, keepdims=True)).sum(1))
    near(out["lse"], lse, 1e-6, 1e-6, "lse")


def test_topk_ties_and_special_cases(orc):
    rng = np.random.default_rng(3)
    T, d, E, K = 40, 128, 6, 3
    X = bf16_bits(rng.standard_normal((T, d)).astype(np.float32))
    # equal logits: ties go to the lower index (moe.cu:60, strict '>')
    out = orc.router(X, np.zeros((E, d), np.uint16), K)
    assert np.all(out["idx"] == np.arange(K))
    near(out["probs"], 1.0 / E, 0, 1e-6, "uniform probs")
    near(out["gate"], 1.0 / K, 0, 1e-6, "uniform gates")
    # E == K: every expert selected, gates equal the softmax
    Wr = bf16_bits(rng.standard_normal((E, d)).astype(np.float32) / 8)
    out = orc.router(X, Wr, E)
    assert np.all(np.sort(out["idx"], 1) == np.arange(E))
    near(out["gate"], np.take_along_axis(out["probs"], out["idx"], 1), 1e-7, 1e-6, "E == K gates")
    # a dominant bias puts that expert first
    bias = np.zeros(E, np.float32)
    bias[E - 1] = 1e4
    out = orc.router(X, Wr, K, bias=bias)
    assert np.all(out["idx"][:, 0] == E - 1)
    # identical router rows tie exactly; the lower index wins
    Wt = Wr.copy()
    Wt[2] = Wt[4]
    bias = np.array([-50, -50, 30, -50, 30, -50], np.float32)
    out = orc.router(X, Wt, 2, bias=bias)
    assert np.all(out["idx"] == np.array([2, 4]))


def _topk_first_max(v, K):
    """K rounds of arg-max with ties to the lower index (argmax's first hit)."""
    v = v.copy()
    rows = np.arange(v.shape[0])
    out = []
    for _ in range(K):
        j = np.argmax(v, 1)
        out.append(j)
        v[rows, j] = -np.inf
    return np.stack(out, 1)


def test_selection_on_logits_vs_fp32_probs():
    """The kernels (and the oracle) rank experts by logit; the reference ranks
    by the fp32 softmax probability (moe.cu:41-63), both with ties to the
    lower index. Softmax is monotone, so the two can differ only where
    distinct logits give one fp32 probability: l - max, exp and the division
    each merge inputs closer than about one ulp of their operands. This
    bounds the case by the absolute logit gap: on random rows the selections
    agree everywhere, and with a planted near-tie straddling the top-k
    boundary (the higher logit on the higher index) they disagree only for
    gaps below 2^-20 when |logit - max| < 8."""
    rng = np.random.default_rng(17)
    E, K = 16, 4

    def probs(l):
        m = l.max(1, keepdims=True)
        e = np.exp((l - m).astype(np.float32)).astype(np.float32)
        return (e / e.sum(1, keepdims=True, dtype=np.float32)).astype(np.float32)

    l = (2.0 * rng.standard_normal((200000, E))).astype(np.float32)
    assert np.array_equal(_topk_first_max(l, K), _topk_first_max(probs(l), K))

    n = 20000
    base = (2.0 * rng.standard_normal((n, E))).astype(np.float32)
    kth = np.sort(base, 1)[:, E - K]  # the K-th largest logit of the row
    base[:, 9] = -1e30
    assert np.abs(base.max(1) - kth).max() < 8
    disagree = {}
    for x in (26, 24, 22, 21, 20, 18, 16):
        l = base.copy()
        l[:, 9] = (kth + np.float32(2.0 ** -x)).astype(np.float32)
        l[:, 9] = np.where(l[:, 9] > kth, l[:, 9], np.nextafter(kth, np.float32(np.inf)))
        a, b = _topk_first_max(l, K), _topk_first_max(probs(l), K)
        disagree[x] = int((~np.all(np.sort(a, 1) == np.sort(b, 1), 1)).sum())
    assert disagree[26] > 0 and disagree[21] > 0  # reachable
    assert disagree[20] == disagree[18] == disagree[16] == 0


# -------------------------------------------------------------- dispatch --

def test_dispatch_brute_force(orc):
    rng = np.random.default_rng(5)
    T, E, K = 1000, 7, 3
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    out = orc.dispatch(idx, E)
    cnt = np.bincount(idx.ravel(), minlength=E)
    assert np.array_equal(out["counts"], cnt)
    assert np.array_equal(out["offsets"], np.concatenate([[0], np.cumsum(cnt)]))
    for e in range(E):
        seg = out["perm"][out["offsets"][e]:out["offsets"][e + 1]]
        assert np.array_equal(seg, np.nonzero((idx == e).any(1))[0])
    r, j = np.nonzero(np.ones_like(idx))
    assert np.array_equal(out["perm"][out["slot_of"][r, j]], r)
    assert np.array_equal(np.sort(out["slot_of"].ravel()), np.arange(T * K))


# ----------------------------------------------------------------- aux/z --

def test_aux_z_closed_forms(orc):
    T, E, K = 64, 8, 2
    probs = np.full((T, E), 1.0 / E, np.float32)
    counts = np.full(E, T * K // E, np.int32)
    aux, z = orc.aux_z(probs, counts, np.zeros(T, np.float32), K)
    assert abs(aux - 1.0) < 1e-6 and z == 0.0
    # all-zero logits: lse = ln E, z = (ln E)^2
    X = bf16_bits(np.random.default_rng(0).standard_normal((T, 128)).astype(np.float32))
    f = orc.forward(X, np.zeros((E, 128), np.uint16),
                    np.zeros((E, 128, 128), np.uint16), np.zeros((E, 128, 128), np.uint16), K, 128)
    assert abs(f["z"] - math.log(E) ** 2) < 1e-5
    assert abs(f["aux"] - 1.0) < 1e-5  # uniform probs, ties -> experts 0..K-1: E*(1/E)*(1) = 1


# ------------------------------------------------- backward: FD and twins --

def _tiny(rng, T, d, E, K, h, bias=True):
    hn = h if h > 0 else d
    X = rng.standard_normal((T, d))
    Wr = rng.standard_normal((E, d)) * 0.7
    Wu = rng.standard_normal((E, hn, d)) / math.sqrt(d)
    Wd = rng.standard_normal((E, d, h)) / math.sqrt(h) if h > 0 else None
    dY = rng.standard_normal((T, d))
    b = rng.standard_normal(E) * 0.3 if bias and E > 1 else None
    return X, Wr, Wu, Wd, dY, b


@pytest.mark.parametrize("T,d,E,K,h", [(6, 8, 4, 2, 6), (5, 8, 4, 2, 0), (4, 8, 1, 1, 0),
                                       (5, 6, 3, 3, 4), (7, 4, 5, 1, 3)])
def test_loss_f64_finite_differences(orc, T, d, E, K, h):
    """Every analytic gradient of the fp64 twin, including the router task
    gradient through the top-k renormalisation that the reference's own tests
    leave unpinned, against central differences."""
    rng = np.random.default_rng(T * 100 + d * 10 + E + h)
    X, Wr, Wu, Wd, dY, b = _tiny(rng, T, d, E, K, h)
    a, zc = (0.7, 0.3) if E > 1 else (0.0, 0.0)
    base = orc.loss_f64(X, Wr, Wu, Wd, dY, K, h, bias=b, aux_coef=a, z_coef=zc)
    eps = 1e-6
    params = {"dX": X, "dWr": Wr, "dW_up": Wu}
    if h > 0:
        params["dW_down"] = Wd
    if E == 1:
        params.pop("dWr")
    for name, arr in params.items():
        flat = arr.reshape(-1)
        for i in range(flat.size):
            old = flat[i]
            flat[i] = old + eps
            hi = orc.loss_f64(X, Wr, Wu, Wd, dY, K, h, bias=b, aux_coef=a, z_coef=zc, grads=False)
            flat[i] = old - eps
            lo = orc.loss_f64(X, Wr, Wu, Wd, dY, K, h, bias=b, aux_coef=a, z_coef=zc, grads=False)
            flat[i] = old
            assert np.array_equal(hi["idx"], base["idx"]) and np.array_equal(lo["idx"], base["idx"])
            fd = (hi["loss"] - lo["loss"]) / (2 * eps)
            near(base[name].reshape(-1)[i], fd, 1e-7, 1e-5, f"{name}[{i}]")


def _bf16_round(a):
    return bf16_to_f32(bf16_bits(np.asarray(a, np.float32))).astype(np.float64)


@pytest.mark.parametrize("T,d,E,K,h", [(40, 16, 4, 2, 24), (33, 16, 5, 3, 0), (20, 16, 1, 1, 0)])
def test_fp32_oracle_matches_fp64_twin(orc, T, d, E, K, h):
    rng = np.random.default_rng(T + d + E + K + h)
    X, Wr, Wu, Wd, dY, b = _tiny(rng, T, d, E, K, h)
    X, Wr, Wu, dY = map(_bf16_round, (X, Wr, Wu, dY))
    Wd = _bf16_round(Wd) if h > 0 else None
    b = None if b is None else b.astype(np.float32).astype(np.float64)
    a, zc = (0.1, 1e-3) if E > 1 else (0.0, 0.0)
    ref = orc.loss_f64(X, Wr, Wu, Wd, dY, K, h, bias=b, aux_coef=a, z_coef=zc)
    u16 = lambda v: bf16_bits(np.asarray(v, np.float32))
    bias32 = None if b is None else b.astype(np.float32)
    got = orc.backward(u16(X), u16(Wr), u16(Wu), u16(Wd) if h > 0 else None, u16(dY), K, h,
                       bias=bias32, aux_coef=a, z_coef=zc)
    fwd = orc.forward(u16(X), u16(Wr), u16(Wu), u16(Wd) if h > 0 else None, K, h, bias=bias32)
    assert np.array_equal(fwd["idx"], ref["idx"])
    assert rel_l2(got["dX"], ref["dX"]) < 1e-5
    assert rel_l2(got["dW_up"], ref["dW_up"]) < 1e-5
    if h > 0:
        assert rel_l2(got["dW_down"], ref["dW_down"]) < 1e-5
    if E > 1:
        assert rel_l2(got["dWr"], ref["dWr"]) < 1e-5
    # forward: loss = <dY, Y> + aux terms, Y from the fp32 oracle
    loss32 = float((dY * fwd["Y"]).sum()) + a * fwd["aux"] + zc * fwd["z"]
    assert abs(loss32 - ref["loss"]) <= 1e-5 * (1 + abs(ref["loss"]))


def test_identical_experts_equal_dense(orc):
    """Restates test_moe_backward (architecture_test.cu:231-264): two identical
    experts, both selected (E=K=2, reference h=0 experts) reproduce the dense
    E=1 layer; summed expert gradients equal the dense gradient."""
    rng = np.random.default_rng(9)
    T, d = 14, 16
    X = bf16_bits(rng.standard_normal((T, d)).astype(np.float32))
    W0 = bf16_bits((rng.standard_normal((d, d)) / 4).astype(np.float32))
    Wr = bf16_bits(rng.standard_normal((2, d)).astype(np.float32) * 0.02)
    dY = bf16_bits(rng.standard_normal((T, d)).astype(np.float32))
    dense_f = orc.forward(X, None, W0[None], None, 1, 0)
    moe_f = orc.forward(X, Wr, np.stack([W0, W0]), None, 2, 0)
    near(moe_f["Y"], dense_f["Y"], 1e-6, 1e-5, "MoE with identical experts differs from dense forward")
    dense_b = orc.backward(X, None, W0[None], None, dY, 1, 0)
    moe_b = orc.backward(X, Wr, np.stack([W0, W0]), None, dY, 2, 0)
    assert rel_l2(moe_b["dW_up"].sum(0), dense_b["dW_up"][0]) < 0.03
    assert rel_l2(moe_b["dX"], dense_b["dX"]) < 0.03
    assert np.abs(moe_b["dWr"]).max() < 1e-5  # s_1 == s_2 -> no router gradient


# ----------------------------------------------------------------- MXFP4 --

def test_mxfp4_known_answers(orc):
    grid = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], np.float32)
    block = np.concatenate([grid, -grid, grid * 0.5, -grid * 0.5]).astype(np.float32)
    packed, scales = orc.mxfp4_quantize(block[None])
    assert scales[0, 0] == 127  # amax 6 -> floor(log2 6) - 2 = 0
    back = orc.mxfp4_dequantize(packed, scales, 32)
    # 0.25 and 0.75 are ties between grid points: they go to the even code
    want = np.where(np.abs(block) == 0.25, 0.0,
                    np.where(np.abs(block) == 0.75, np.sign(block), block)).astype(np.float32)
    assert np.array_equal(back[0], want)
    # exact grid values round-trip exactly
    exact = np.concatenate([grid, -grid, grid, -grid]).astype(np.float32) * 4
    p2, s2 = orc.mxfp4_quantize(exact[None])
    assert s2[0, 0] == 127 + 2
    assert np.array_equal(orc.mxfp4_dequantize(p2, s2, 32)[0], exact)
    # ties go to the even code: 0.25 -> 0, 0.75 -> 1, 1.25 -> 1, 2.5 -> 2, 5 -> 4
    ties = np.zeros(32, np.float32)
    ties[:6] = [0.25, 0.75, 1.25, 1.75, 2.5, 5.0]
    ties[31] = 6.0
    p3, s3 = orc.mxfp4_quantize(ties[None])
    d3 = orc.mxfp4_dequantize(p3, s3, 32)[0]
    assert list(d3[:6]) == [0.0, 1.0, 1.0, 2.0, 2.0, 4.0]


def test_mxfp4_round_trip_and_error_bound(orc):
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((64, 256)) / 16).astype(np.float32)
    packed, scales = orc.mxfp4_quantize(w)
    deq = orc.mxfp4_dequantize(packed, scales, 256)
    p2, s2 = orc.mxfp4_quantize(deq)
    assert np.array_equal(p2, packed) and np.array_equal(s2, scales)  # idempotent
    # inside the grid (|w| <= 6*2^s) the error is at most half a spacing
    # (spacing <= 2 * 2^s); above it values saturate to 6*2^s and |w| < 8*2^s
    scale = np.exp2(scales.astype(np.float64) - 127).repeat(32, axis=1)
    err = np.abs(deq.astype(np.float64) - w)
    inside = np.abs(w) <= 6 * scale
    assert np.all(err[inside] <= scale[inside] + 1e-12)
    assert np.all(np.abs(deq[~inside]) == 6 * scale[~inside])
    assert np.all(err[~inside] < 2 * scale[~inside])


# --------------------------------------------------- torch-autograd fixture --

def test_torch_autograd_fixture(orc):
    """Independent third-party implementation: torch CPU autograd in fp64 on
    a tiny case (tests/golden/make_golden.py) -- the check the reference's
    ARCHITECTURE.md:74-75 describes and whose test was deleted."""
    path = os.path.join(GOLDEN, "tiny_autograd.npz")
    g = np.load(path, allow_pickle=False)
    for tag in ("h", "h0"):
        X, Wr, Wu, dY, bias = (g[f"{tag}_{k}"] for k in ("X", "Wr", "Wu", "dY", "bias"))
        Wd = g[f"{tag}_Wd"] if f"{tag}_Wd" in g else None
        K, h = int(g[f"{tag}_K"]), int(g[f"{tag}_h"])
        a, zc = float(g[f"{tag}_aux"]), float(g[f"{tag}_z"])
        ref = orc.loss_f64(X, Wr, Wu, Wd, dY, K, h, bias=bias, aux_coef=a, z_coef=zc)
        near(ref["loss"], g[f"{tag}_loss"], 1e-10, 1e-10, "loss")
        for name in ("dX", "dWr", "dW_up") + (("dW_down",) if h > 0 else ()):
            near(ref[name], g[f"{tag}_{name}"], 1e-10, 1e-8, f"{tag} {name}")
