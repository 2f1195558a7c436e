"""GPU parity of the LayerNorm-fronted block (tmt_moe_forward_ln /
tmt_moe_backward_ln) against the oracle, through the C ABI.

The reference's recurrent block runs layernorm_fwd, then moe_forward on its
output, and in the backward moe_backward, then layernorm_bwd on the bf16
gradient it produced (tmt-cuda/src/model.cu:509-514, 674-680). The oracle
composes the same steps: orc.layernorm -> orc.forward/backward on H ->
round dX to bf16 -> orc.layernorm_bwd.

Bars:
  * H, the row mean and 1/std bit-identical to the oracle (fixed summation
    order), and therefore the routing bit-exact as in the plain block;
  * Y, dS, dGamma, dBeta and the weight gradients within 1e-2 relative L2.
"""
import sys

import numpy as np
import pytest
import torch

import tmt_moe
from synthetic import CONFIGS, bf16_bits, bf16_to_f32, make_case
from test_gpu_parity import LOGIT_ATOL, LOGIT_RTOL, near

pytestmark = pytest.mark.gpu

REL_L2 = 1e-2


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def dev(u16):
    return torch.from_numpy(np.ascontiguousarray(u16).view(np.int16)).cuda().view(torch.bfloat16)


def host_f32(t):
    return bf16_to_f32(t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16))


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def ln_inputs(X, seed):
    """LayerNorm input with per-row offsets and scales (so the normalisation
    matters), and non-trivial gamma / beta."""
    rng = np.random.default_rng(seed)
    T, d = X.shape
    scale = np.exp(rng.uniform(-1.0, 1.5, (T, 1))).astype(np.float32)
    shift = rng.standard_normal((T, 1)).astype(np.float32)
    S = bf16_bits(bf16_to_f32(X) * scale + shift)
    gamma = (1.0 + 0.2 * rng.standard_normal(d)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(d)).astype(np.float32)
    return S, gamma, beta


def run_gpu_ln(case, S, gamma, beta, K, h, Y0, aux, z):
    T, d = S.shape
    E = case["W_up"].shape[0]
    hn = h if h > 0 else d
    m = tmt_moe.MoE(max(T, 1), d, E, K, h)
    try:
        Sd, g_d, b_d = dev(S), torch.from_numpy(gamma).cuda(), torch.from_numpy(beta).cuda()
        Wr = dev(case["Wr"])
        Wu = dev(case["W_up"])
        Wd = dev(case["W_down"]) if h > 0 else None
        Y = dev(Y0)
        m.forward_ln(Sd, g_d, b_d, Wr, Wu, Wd, Y, beta=1.0)
        out = {"Y": host_f32(Y)}
        out.update(m.routing())
        out.update(m.norm())
        out["aux"], out["z"], out["counts"] = m.stats()
        nan = float("nan")
        dS = torch.full((T, d), nan, dtype=torch.bfloat16, device="cuda")
        dG = torch.full((d,), nan, dtype=torch.float32, device="cuda")
        dB = torch.full((d,), nan, dtype=torch.float32, device="cuda")
        dWr = torch.full((E, d), nan, dtype=torch.float32, device="cuda") if E > 1 else None
        dWu = torch.full((E, hn, d), nan, dtype=torch.float32, device="cuda")
        dWd = torch.full((E, d, h), nan, dtype=torch.float32, device="cuda") if h > 0 else None
        m.backward_ln(dev(case["dY"]), Sd, g_d, Wr, Wu, Wd, dS, dG, dB, dWr, dWu, dWd, aux, z)
        torch.cuda.synchronize()
        out.update(dS=host_f32(dS), dgamma=dG.cpu().numpy(), dbeta=dB.cpu().numpy(),
                   dW_up=dWu.cpu().numpy())
        out["dWr"] = dWr.cpu().numpy() if E > 1 else None
        out["dW_down"] = dWd.cpu().numpy() if h > 0 else None
    finally:
        m.close()
    return out


def oracle_ln(orc, case, S, gamma, beta, K, h, Y0, aux, z):
    ln = orc.layernorm(S, gamma, beta)
    H = ln["H"]
    r = orc.forward(H, case["Wr"], case["W_up"], case["W_down"], K, h, Y_in=Y0, beta=1.0)
    r.update(orc.backward(H, case["Wr"], case["W_up"], case["W_down"], case["dY"], K, h,
                          aux_coef=aux, z_coef=z))
    dH = bf16_to_f32(bf16_bits(r["dX"]))  # the block hands LayerNorm a bf16 gradient
    r.update(ln)
    r.update(orc.layernorm_bwd(S, dH, gamma, ln["mean"], ln["rstd"]))
    return r


def check_all(g, r, E, h):
    assert np.array_equal(g["H"], r["H"]), "LayerNorm output is not bit-identical"
    assert np.array_equal(g["mean"].view(np.uint32), r["mean"].view(np.uint32)), "row means differ"
    assert np.array_equal(g["rstd"].view(np.uint32), r["rstd"].view(np.uint32)), "row 1/std differ"
    assert np.array_equal(g["idx"], r["idx"]), "top-k indices differ"
    if E > 1:
        # bit-identical where the LayerNorm runs inside the router (its
        # canonical order); where it does not, the routed batch's logits come
        # from the matrix cores (tolerance, picks exact)
        near(g["logits"], r["logits"], LOGIT_ATOL, LOGIT_RTOL, "logits")
    assert np.array_equal(g["offsets"], r["offsets"])
    assert np.array_equal(g["perm"], r["perm"])
    assert np.array_equal(g["counts"], r["counts"])
    names = ["Y", "dS", "dgamma", "dbeta", "dW_up"] + (["dW_down"] if h > 0 else []) + \
        (["dWr"] if E > 1 else [])
    for n in names:
        assert np.isfinite(g[n]).all(), f"{n} has unwritten/non-finite entries"
        err = rel_l2(g[n], r[n])
        say(f"  {n}: rel-L2 {err:.2e}")
        assert err <= REL_L2, f"{n} rel-L2 {err:.3e} > {REL_L2}"


@pytest.mark.parametrize("T,d,E,K,h", [
    (300, 256, 4, 2, 1024),    # a few 64-row workgroups of the fused dGamma/dBeta partials
    (1237, 384, 8, 2, 256),    # ragged T, d not a multiple of 512
    (520, 1088, 4, 2, 128),    # d > 512: three row passes per lane, the last partial
    (520, 1088, 16, 4, 128),   # LayerNorm inside the router: 4 chunk slots, the third partial, the fourth empty
    (777, 256, 1, 1, 0),       # reference dense path (experts=1, no router)
    (700, 512, 16, 4, 0),      # reference single-linear experts
    (5, 192, 5, 2, 320),       # decode-sized: fused router, weight-streaming GEMMs
    (64, 1024, 16, 4, 512),    # largest decode batch, c3 width
    (2100, 2048, 12, 2, 128),  # widest row of the scatter-fused backward (4 passes per lane)
    (300, 2560, 4, 2, 128),    # d > 2048: separate two-pass LayerNorm backward
    (200, 2048, 32, 4, 128),   # E*d beyond the LDS-staged router: fused scatter reads Wr from memory
    (160, 2560, 16, 4, 0),     # the same on the separate LayerNorm backward, reference experts
])
def test_layernorm_block_against_oracle(orc, T, d, E, K, h):
    say(f"layernorm block T={T} d={d} E={E} K={K} h={h} fwd+bwd")
    case = make_case(T, d, E, K, h, seed=3 * T + d)
    S, gamma, beta = ln_inputs(case["X"], seed=T)
    Y0 = bf16_bits(np.random.default_rng(d).standard_normal((T, d)).astype(np.float32))
    aux, z = (0.1, 1e-3) if E > 1 else (0.0, 0.0)
    g = run_gpu_ln(case, S, gamma, beta, K, h, Y0, aux, z)
    r = oracle_ln(orc, case, S, gamma, beta, K, h, Y0, aux, z)
    check_all(g, r, E, h)


def test_layernorm_constant_rows_and_extreme_scales(orc):
    say("layernorm block: constant rows, 1e-3 and 1e3 scaled rows")
    T, d, E, K, h = 96, 256, 4, 2, 128
    case = make_case(T, d, E, K, h, seed=5)
    S, gamma, beta = ln_inputs(case["X"], seed=6)
    X = bf16_to_f32(S)
    X[0::3] = X[0::3, :1]           # constant rows: H = beta exactly
    X[1::3] *= 1e-3
    X[2::3] *= 1e3
    S = bf16_bits(X)
    Y0 = np.zeros((T, d), np.uint16)
    g = run_gpu_ln(case, S, gamma, beta, K, h, Y0, 0.1, 1e-3)
    r = oracle_ln(orc, case, S, gamma, beta, K, h, Y0, 0.1, 1e-3)
    assert np.array_equal(g["H"][0::3], np.broadcast_to(bf16_bits(beta), (T // 3, d)))
    check_all(g, r, E, h)


def test_layernorm_empty_batch():
    say("layernorm block T=0")
    d, E, K, h = 128, 4, 2, 128
    m = tmt_moe.MoE(16, d, E, K, h)
    try:
        case = make_case(16, d, E, K, h, seed=2)
        S = torch.zeros(0, d, dtype=torch.bfloat16, device="cuda")
        g_d = torch.ones(d, device="cuda")
        b_d = torch.zeros(d, device="cuda")
        Wr, Wu, Wd = dev(case["Wr"]), dev(case["W_up"]), dev(case["W_down"])
        Y = torch.zeros(0, d, dtype=torch.bfloat16, device="cuda")
        m.forward_ln(S, g_d, b_d, Wr, Wu, Wd, Y)
        dG = torch.full((d,), float("nan"), device="cuda")
        dB = torch.full((d,), float("nan"), device="cuda")
        dWr = torch.full((E, d), float("nan"), device="cuda")
        dWu = torch.full((E, h, d), float("nan"), device="cuda")
        dWd = torch.full((E, d, h), float("nan"), device="cuda")
        m.backward_ln(Y, S, g_d, Wr, Wu, Wd, S, dG, dB, dWr, dWu, dWd, 0.1, 1e-3)
        torch.cuda.synchronize()
        for t in (dG, dB, dWr, dWu, dWd):
            assert torch.count_nonzero(t).item() == 0
    finally:
        m.close()


def test_backward_ln_needs_forward_ln():
    say("layernorm block: backward_ln after a plain forward is rejected")
    T, d, E, K, h = 32, 128, 4, 2, 128
    case = make_case(T, d, E, K, h, seed=4)
    m = tmt_moe.MoE(T, d, E, K, h)
    try:
        X, Wr, Wu, Wd = dev(case["X"]), dev(case["Wr"]), dev(case["W_up"]), dev(case["W_down"])
        Y = torch.zeros(T, d, dtype=torch.bfloat16, device="cuda")
        m.forward(X, Wr, Wu, Wd, Y)
        g_d = torch.ones(d, device="cuda")
        dG = torch.zeros(d, device="cuda")
        dWr = torch.zeros(E, d, device="cuda")
        dWu = torch.zeros(E, h, d, device="cuda")
        dWd = torch.zeros(E, d, h, device="cuda")
        with pytest.raises(tmt_moe.MoeError) as ei:
            m.backward_ln(Y, X, g_d, Wr, Wu, Wd, Y, dG, dG, dWr, dWu, dWd)
        assert ei.value.code == -4
        with pytest.raises(tmt_moe.MoeError):
            m.norm()
        torch.cuda.synchronize()
    finally:
        m.close()


def test_plain_backward_after_forward_ln_is_rejected():
    say("layernorm block: a plain backward after forward_ln is rejected")
    T, d, E, K, h = 32, 128, 4, 2, 128
    case = make_case(T, d, E, K, h, seed=5)
    m = tmt_moe.MoE(T, d, E, K, h)
    try:
        S, Wr, Wu, Wd = dev(case["X"]), dev(case["Wr"]), dev(case["W_up"]), dev(case["W_down"])
        Y = torch.zeros(T, d, dtype=torch.bfloat16, device="cuda")
        g_d, b_d = torch.ones(d, device="cuda"), torch.zeros(d, device="cuda")
        m.forward_ln(S, g_d, b_d, Wr, Wu, Wd, Y)
        dX = torch.zeros_like(S)
        dWr = torch.zeros(E, d, device="cuda")
        dWu = torch.zeros(E, h, d, device="cuda")
        dWd = torch.zeros(E, d, h, device="cuda")
        with pytest.raises(tmt_moe.MoeError) as ei:
            m.backward(Y, S, Wr, Wu, Wd, dX, dWr, dWu, dWd)
        assert ei.value.code == -4
        torch.cuda.synchronize()
    finally:
        m.close()


@pytest.mark.parametrize("T,d", [(1, 64), (777, 384), (4096, 1024), (300, 2560), (0, 128)])
def test_standalone_layernorm_against_oracle(orc, T, d):
    """tmt_moe_layernorm_forward / _backward (the reference's layernorm_fwd /
    layernorm_bwd): H, mean, rstd bit-identical; dS, dGamma, dBeta within
    1e-2 rel-L2 of the oracle on the same bf16 dH."""
    say(f"standalone layernorm T={T} d={d}")
    rng = np.random.default_rng(T + d)
    X = bf16_bits(rng.standard_normal((max(T, 1), d)).astype(np.float32))[:T]
    S, gamma, beta = ln_inputs(X, seed=d)
    dH = bf16_bits(rng.standard_normal((T, d)).astype(np.float32))
    Sd = dev(S)
    g_d, b_d = torch.from_numpy(gamma).cuda(), torch.from_numpy(beta).cuda()
    H = torch.empty(T, d, dtype=torch.bfloat16, device="cuda")
    mean = torch.empty(T, device="cuda")
    rstd = torch.empty(T, device="cuda")
    tmt_moe.layernorm_forward(Sd, g_d, b_d, H, mean, rstd)
    ws = torch.empty(tmt_moe.layernorm_workspace_size(T, d), dtype=torch.uint8, device="cuda")
    dS = torch.full((T, d), float("nan"), dtype=torch.bfloat16, device="cuda")
    dG = torch.full((d,), float("nan"), device="cuda")
    dB = torch.full((d,), float("nan"), device="cuda")
    tmt_moe.layernorm_backward(Sd, dev(dH), g_d, mean, rstd, dS, dG, dB, ws)
    torch.cuda.synchronize()
    ref = orc.layernorm(S, gamma, beta)
    Hh = H.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(Hh, ref["H"]), "H is not bit-identical"
    assert np.array_equal(mean.cpu().numpy().view(np.uint32), ref["mean"].view(np.uint32))
    assert np.array_equal(rstd.cpu().numpy().view(np.uint32), ref["rstd"].view(np.uint32))
    rb = orc.layernorm_bwd(S, bf16_to_f32(dH), gamma, ref["mean"], ref["rstd"])
    got = {"dS": host_f32(dS), "dgamma": dG.cpu().numpy(), "dbeta": dB.cpu().numpy()}
    for n in ("dS", "dgamma", "dbeta"):
        assert np.isfinite(got[n]).all(), n
        if T == 0:
            assert not got[n].any(), n
            continue
        err = rel_l2(got[n], rb[n])
        say(f"  {n}: rel-L2 {err:.2e}")
        assert err <= REL_L2, f"{n} rel-L2 {err:.3e}"


def test_c3_full_size_layernorm_block(orc):
    """At the c3 size: H bit-exact against the oracle LayerNorm, routing
    bit-exact against the oracle router on H, and the LayerNorm-fronted block
    equal to the plain block on H (at this batch size both route H on the
    matrix cores, the LayerNorm running as its own launch first): the same
    picks, Y and the weight gradients within 1e-3 relative L2, and the
    LayerNorm backward against the oracle's."""
    cfg = CONFIGS["c3"]
    T, d, E, K, h = (cfg[k] for k in ("T", "d", "E", "K", "h"))
    say(f"c3 layernorm block T={T} d={d} E={E} K={K} h={h} fwd+bwd")
    case = make_case(**cfg)
    S, gamma, beta = ln_inputs(case["X"], seed=11)
    aux, z = cfg["aux"], cfg["z"]
    Wr, Wu, Wd = dev(case["Wr"]), dev(case["W_up"]), dev(case["W_down"])
    Sd, g_d, b_d = dev(S), torch.from_numpy(gamma).cuda(), torch.from_numpy(beta).cuda()
    dY = dev(case["dY"])

    def grads():
        return (torch.empty(E, d, device="cuda"), torch.empty(E, h, d, device="cuda"),
                torch.empty(E, d, h, device="cuda"))

    m = tmt_moe.MoE(T, d, E, K, h)
    p = tmt_moe.MoE(T, d, E, K, h)
    try:
        Y = torch.zeros(T, d, dtype=torch.bfloat16, device="cuda")
        m.forward_ln(Sd, g_d, b_d, Wr, Wu, Wd, Y)
        nm = m.norm()
        routing = m.routing()
        dS = torch.empty(T, d, dtype=torch.bfloat16, device="cuda")
        dG, dB = torch.empty(d, device="cuda"), torch.empty(d, device="cuda")
        a = grads()
        m.backward_ln(dY, Sd, g_d, Wr, Wu, Wd, dS, dG, dB, *a, aux, z)
        # the plain block on the same H
        H = dev(nm["H"])
        Y2 = torch.zeros(T, d, dtype=torch.bfloat16, device="cuda")
        p.forward(H, Wr, Wu, Wd, Y2)
        dH = torch.empty(T, d, dtype=torch.bfloat16, device="cuda")
        b = grads()
        p.backward(dY, H, Wr, Wu, Wd, dH, *b, aux, z)
        torch.cuda.synchronize()
        plain = p.routing()
        for key in ("idx", "perm", "offsets"):
            assert np.array_equal(routing[key], plain[key]), f"{key} differs from the plain block"
        err = rel_l2(host_f32(Y), host_f32(Y2))
        say(f"  Y against the plain block: rel-L2 {err:.2e}")
        assert err <= 1e-3
        for x, y, n in zip(a, b, ("dWr", "dW_up", "dW_down")):
            err = rel_l2(x.cpu().numpy(), y.cpu().numpy())
            say(f"  {n} against the plain block: rel-L2 {err:.2e}")
            assert err <= 1e-3, f"{n} differs from the plain block"
        dH_host = host_f32(dH)
        got = {"dS": host_f32(dS), "dgamma": dG.cpu().numpy(), "dbeta": dB.cpu().numpy()}
    finally:
        m.close()
        p.close()
    ln = orc.layernorm(S, gamma, beta)
    assert np.array_equal(nm["H"], ln["H"]), "LayerNorm output is not bit-identical"
    assert np.array_equal(nm["rstd"].view(np.uint32), ln["rstd"].view(np.uint32))
    rr = orc.router(ln["H"], case["Wr"], K)
    assert np.array_equal(routing["idx"], rr["idx"])
    near(routing["logits"], rr["logits"], LOGIT_ATOL, LOGIT_RTOL, "logits")
    ref = orc.layernorm_bwd(S, dH_host, gamma, ln["mean"], ln["rstd"])
    for n in ("dS", "dgamma", "dbeta"):
        err = rel_l2(got[n], ref[n])
        say(f"  {n}: rel-L2 {err:.2e}")
        assert err <= REL_L2, f"{n} rel-L2 {err:.3e}"


@pytest.mark.parametrize("T,d,E,norm_launches", [
    (300, 256, 4, 0),     # routed batch: the router normalises its rows itself
    (2100, 2048, 12, 0),  # the widest fused row (4 chunks of 512 per lane)
    (40, 256, 4, 1),      # decode-sized batch: separate LayerNorm launch
    (300, 2560, 4, 1),    # d > 2048: separate LayerNorm launch
    (32768, 256, 4, 1),   # one 128-row group per CU: separate LayerNorm launch, matrix-core router over H
])
def test_layernorm_forward_placement(T, d, E, norm_launches):
    """Which kernel runs the LayerNorm forward: the phase profile counts the
    separate LayerNorm launches; H and the statistics are checked bit for bit
    against the oracle by the block tests above for each of these paths."""
    say(f"layernorm placement T={T} d={d} E={E}: {norm_launches} LayerNorm launch(es)")
    K, h = 2, 128
    case = make_case(T, d, E, K, h, seed=T + d)
    S, gamma, beta = ln_inputs(case["X"], seed=1)
    m = tmt_moe.MoE(T, d, E, K, h)
    try:
        Wr, Wu, Wd = dev(case["Wr"]), dev(case["W_up"]), dev(case["W_down"])
        Y = torch.zeros(T, d, dtype=torch.bfloat16, device="cuda")
        m.set_profiling(True)
        m.profile(reset=True)
        m.forward_ln(dev(S), torch.from_numpy(gamma).cuda(), torch.from_numpy(beta).cuda(), Wr, Wu, Wd, Y)
        prof = m.profile(reset=True)
        m.set_profiling(False)
        assert prof["norm"][1] == norm_launches
        assert prof["router"][1] + prof["gemm_up"][1] >= 1
    finally:
        m.close()
