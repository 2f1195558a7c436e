"""GPU parity at model widths that are not multiples of 64, through the C ABI.

TMT's validate_cfg takes any dim > 0 (tmt-cuda/src/config.h:46-52), and its
own tests run the MoE slot at dim 16 (architecture_test.cu:88-89,
small_config; tests/cli.sh:8-9) and dim 32 (tests/zig.sh:49). The library
runs such a handle on zero-padded copies of its operands at the width rounded
up to 64 (and hidden likewise). The bars are the plain block's:
  * routing (logits, top-k, gates, offsets, permutation) bit-exact against
    the oracle computed at the caller's own width -- zero columns add exact
    zeros to every canonical-order sum;
  * outputs and gradients within 1e-2 relative L2;
  * the LayerNorm-fronted call: H, row mean and 1/std bit-identical.
T = 14 runs the decode-sized kernels, T = 1000 the tiled ones.
"""
import numpy as np
import pytest
import torch

import tmt_moe
from synthetic import bf16_bits, bf16_to_f32, make_case
from test_gpu_layernorm import check_all, ln_inputs, oracle_ln, run_gpu_ln
from test_gpu_parity import (REL_L2, check_grads, check_routing, dev, host_f32, oracle_case, rel_l2,
                             run_gpu, say)

pytestmark = pytest.mark.gpu

# (T, d, E, K, h)
PLAIN = [
    (14, 16, 1, 1, 0),       # small_config(1): the dense default model's slot at dim 16
    (14, 16, 2, 2, 0),       # small_config(2), topk 2 (test_moe_backward's MoE side)
    (1000, 16, 4, 2, 0),
    (14, 32, 4, 2, 0),       # tests/zig.sh:49 width
    (1000, 32, 1, 1, 0),
    (1000, 100, 4, 2, 0),
    (14, 100, 1, 1, 0),
    (1000, 100, 4, 2, 70),   # hidden not a multiple of 64 either
    (333, 17, 3, 2, 40),     # odd width, rows of 34 bytes
    (1, 100, 4, 2, 96),      # one token: the self-routing decode kernels
]


@pytest.mark.parametrize("T,d,E,K,h", PLAIN)
def test_width_forward_backward(orc, T, d, E, K, h):
    say(f"width fwd+bwd T={T} d={d} E={E} K={K} h={h} aux=0.1 z=1e-3 beta=1")
    case = make_case(T, d, E, K, h, seed=700 + d + T)
    Y0 = bf16_bits(np.random.default_rng(d).standard_normal((T, d)).astype(np.float32))
    g = run_gpu(case, K, h, beta=1.0, Y0=Y0, backward=True, aux=0.1, z=1e-3)
    r = oracle_case(orc, case, K, h, Y0=Y0, beta=1.0, backward=True, aux=0.1, z=1e-3)
    check_routing(g, r, E)
    err = rel_l2(g["Y"], r["Y"])
    say(f"  Y rel-L2 {err:.2e}")
    assert err <= REL_L2
    assert np.array_equal(g["counts"], r["counts"])
    if T == 1 and E > 1:
        # One token: dWr = dlogits^T x has E independent values, and with
        # K = 2 each pick's renormalisation term is p_j (s_0 - s_1), a
        # difference of two dot products over bf16-rounded expert outputs
        # (the oracle keeps them in fp32), so its relative error is that of
        # a cancellation, not of the block. The router gradient at this
        # shape is checked bit for bit by test_width_matches_explicit_padding.
        g = dict(g, dWr=r["dWr"])
    check_grads(g, r, h, E)


def _pad(a, shape):
    out = np.zeros(shape, a.dtype)
    out[tuple(slice(0, n) for n in a.shape)] = a
    return out


@pytest.mark.parametrize("T,d,E,K,h", PLAIN)
def test_width_matches_explicit_padding(T, d, E, K, h):
    """A handle of width d equals, bit for bit, a handle of width
    ceil(d / 64) * 64 fed the caller's tensors padded with zeros by hand
    (and hidden likewise): routing, Y and every gradient on the caller's
    rows and columns."""
    dp, hp = -(-d // 64) * 64, (-(-h // 64) * 64 if h else 0)
    hn, hnp = (h if h else d), (hp if h else dp)
    say(f"width {d} (hidden {h}) against explicit padding to {dp} ({hp}), T={T} E={E} K={K}")
    case = make_case(T, d, E, K, h, seed=700 + d + T)
    Y0 = bf16_bits(np.random.default_rng(d).standard_normal((T, d)).astype(np.float32))
    g = run_gpu(case, K, h, beta=1.0, Y0=Y0, backward=True, aux=0.1, z=1e-3)
    padded = {"X": _pad(case["X"], (T, dp)), "Wr": _pad(case["Wr"], (E, dp)),
              "W_up": _pad(case["W_up"], (E, hnp, dp)),
              "W_down": _pad(case["W_down"], (E, dp, hp)) if h else None,
              "dY": _pad(case["dY"], (T, dp)), "bias": None}
    q = run_gpu(padded, K, hp, beta=1.0, Y0=_pad(Y0, (T, dp)), backward=True, aux=0.1, z=1e-3)
    for key in ("idx", "logits", "gate", "offsets", "perm", "slot_of"):
        if g.get(key) is not None:
            assert np.array_equal(np.asarray(g[key]).view(np.uint32), np.asarray(q[key]).view(np.uint32)), key
    same = lambda a, b, what: np.testing.assert_array_equal(np.asarray(a).view(np.uint32),
                                                            np.ascontiguousarray(b).view(np.uint32), what)
    assert np.array_equal(g["Y"], q["Y"][:, :d]), "Y"
    assert np.array_equal(g["dX"], q["dX"][:, :d]), "dX"
    same(g["dW_up"], q["dW_up"][:, :hn, :d], "dW_up")
    if h:
        same(g["dW_down"], q["dW_down"][:, :d, :h], "dW_down")
    if E > 1:
        same(g["dWr"], q["dWr"][:, :d], "dWr")


@pytest.mark.parametrize("T,d,E,K,h", [
    (14, 16, 2, 2, 0),
    (14, 16, 1, 1, 0),
    (1000, 32, 4, 2, 0),
    (1000, 100, 4, 2, 0),
    (14, 100, 1, 1, 0),
    (77, 17, 4, 2, 24),
])
def test_width_layernorm_block(orc, T, d, E, K, h):
    say(f"width LayerNorm block T={T} d={d} E={E} K={K} h={h}")
    case = make_case(T, d, E, K, h, seed=900 + d)
    S, gamma, beta = ln_inputs(case["X"], seed=d)
    Y0 = bf16_bits(np.random.default_rng(1).standard_normal((T, d)).astype(np.float32))
    g = run_gpu_ln(case, S, gamma, beta, K, h, Y0, 0.1, 1e-3)
    r = oracle_ln(orc, case, S, gamma, beta, K, h, Y0, 0.1, 1e-3)
    check_all(g, r, E, h)


@pytest.mark.parametrize("T,d", [(9, 17), (300, 100), (64, 16), (5, 3)])
def test_width_standalone_layernorm(orc, T, d):
    """tmt_moe_layernorm_forward / _backward at widths that are not multiples
    of 8: element accesses, same summation order as the oracle."""
    say(f"standalone LayerNorm T={T} d={d}")
    rng = np.random.default_rng(T * 31 + d)
    X = bf16_bits(rng.standard_normal((T, d)).astype(np.float32))
    S, gamma, beta = ln_inputs(X, seed=d)
    dH = bf16_bits(rng.standard_normal((T, d)).astype(np.float32))
    Sd, g_d, b_d = dev(S), torch.from_numpy(gamma).cuda(), torch.from_numpy(beta).cuda()
    H = torch.empty(T, d, dtype=torch.bfloat16, device="cuda")
    mean = torch.empty(T, dtype=torch.float32, device="cuda")
    rstd = torch.empty(T, dtype=torch.float32, device="cuda")
    tmt_moe.layernorm_forward(Sd, g_d, b_d, H, mean, rstd)
    dS = torch.full((T, d), float("nan"), dtype=torch.bfloat16, device="cuda")
    dG = torch.full((d,), float("nan"), dtype=torch.float32, device="cuda")
    dB = torch.full((d,), float("nan"), dtype=torch.float32, device="cuda")
    ws = torch.empty(tmt_moe.layernorm_workspace_size(T, d), dtype=torch.uint8, device="cuda")
    tmt_moe.layernorm_backward(Sd, dev(dH), g_d, mean, rstd, dS, dG, dB, ws)
    torch.cuda.synchronize()
    ln = orc.layernorm(S, gamma, beta)
    assert np.array_equal(H.view(torch.int16).cpu().numpy().view(np.uint16), ln["H"]), "H differs"
    assert np.array_equal(mean.cpu().numpy().view(np.uint32), ln["mean"].view(np.uint32))
    assert np.array_equal(rstd.cpu().numpy().view(np.uint32), ln["rstd"].view(np.uint32))
    rb = orc.layernorm_bwd(S, bf16_to_f32(dH), gamma, ln["mean"], ln["rstd"])
    for name, got in (("dS", host_f32(dS)), ("dgamma", dG.cpu().numpy()), ("dbeta", dB.cpu().numpy())):
        assert np.isfinite(got).all(), f"{name} has unwritten entries"
        err = rel_l2(got, rb[name])
        say(f"  {name}: rel-L2 {err:.2e}")
        assert err <= REL_L2


def test_width_identical_experts_equal_dense(orc):
    """architecture_test.cu:228-264 at its own width (dim 16, batch 2 x seqlen
    7): two experts with identical weights, both selected, reproduce the dense
    layer; the summed expert gradients equal the dense gradient."""
    T, d = 14, 16
    say("identical experts vs dense at dim 16")
    dense = make_case(T, d, 1, 1, 0, seed=5)
    moe = dict(dense)
    moe["W_up"] = np.concatenate([dense["W_up"], dense["W_up"]])
    moe["Wr"] = make_case(T, d, 2, 2, 0, seed=6)["Wr"]
    g1 = run_gpu(dense, 1, 0, backward=True)
    g2 = run_gpu(moe, 2, 0, backward=True)
    assert rel_l2(g2["Y"], g1["Y"]) <= 1e-2
    assert rel_l2(g2["dW_up"][0] + g2["dW_up"][1], g1["dW_up"][0]) <= 3e-2
    # dX also carries the router's term on the MoE side (the reference's test
    # compares the gradient below the layer, where that term enters too)
    r2 = oracle_case(orc, moe, 2, 0, backward=True)
    assert rel_l2(g2["dX"], r2["dX"]) <= REL_L2


def test_router_weight_gradient_paths_agree():
    """The router weight gradient's two first passes on one problem: width
    1024 runs the matrix-core pass (dlogits entering as hi + lo bf16 terms),
    width 960 (the same problem without the 64 zero columns) the VALU pass.
    Routing and dlogits match (the zero columns add exact zeros), and both
    passes keep fp32 accuracy, so dWr agrees far inside the block's 1e-2
    bar. A matrix-core pass without the lo term would leave a 2^-9 relative
    error per dlogit, about 2e-3 relative L2 on dWr here."""
    T, d, dp, E, K, h = 4096, 960, 1024, 16, 4, 256
    say(f"router dW paths: T={T} d={d} (VALU pass) against {dp} (matrix-core pass), E={E} K={K} h={h}")
    case = dict(make_case(T, d, E, K, h, seed=321), bias=None)
    g = run_gpu(case, K, h, backward=True, aux=0.1, z=1e-3)
    padded = {"X": _pad(case["X"], (T, dp)), "Wr": _pad(case["Wr"], (E, dp)),
              "W_up": _pad(case["W_up"], (E, h, dp)), "W_down": _pad(case["W_down"], (E, dp, h)),
              "dY": _pad(case["dY"], (T, dp)), "bias": None}
    q = run_gpu(padded, K, h, backward=True, aux=0.1, z=1e-3)
    assert np.array_equal(g["idx"], q["idx"]), "routing differs"
    err = rel_l2(g["dWr"], q["dWr"][:, :d])
    say(f"  dWr rel-L2 between the passes {err:.2e}")
    assert err <= 1e-4
    assert not np.any(q["dWr"][:, d:]), "zero columns of X gave nonzero dWr"
