"""GPU parity of the MXFP4 expert path (config c5) through the C ABI, for
both MXFP4 formats: WEIGHTS_MXFP4 (weights expanded to bf16, bf16
activations) and WEIGHTS_MXFP4_MX (scaled FP6 x FP4 MFMA with the
activations rounded to two MXFP6 terms).

Reference: the same block with the exactly dequantised weights -- the CPU
oracle at a reduced token count and fp32 torch on the GPU at the full c5
size, with routing first matched bit for bit against the oracle router.
Tolerance 2e-2 relative L2 (the c5 contract). The MX format's own
activation rounding is about 1e-3 (tests/test_mxfp4_host.py pins the
scheme on the host); the tests also hold it to 5e-3 against the exact
format's output."""
import sys

import numpy as np
import pytest
import torch

import tmt_moe
from synthetic import CONFIGS, bf16_bits, bf16_to_f32, make_case, mxfp4_experts
from torch_ref import moe_reference

pytestmark = pytest.mark.gpu
TOL = 2e-2


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def dev16(u16):
    return torch.from_numpy(np.ascontiguousarray(u16).view(np.int16)).cuda().view(torch.bfloat16)


def dev8(u8):
    return torch.from_numpy(np.ascontiguousarray(u8)).cuda()


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


FORMATS = [tmt_moe.WEIGHTS_MXFP4, tmt_moe.WEIGHTS_MXFP4_MX, tmt_moe.WEIGHTS_MXFP4_MX_PLANES]


def planes(codes):
    """Per-expert K-plane copies of stacked codes [E, N, K/2] (the layout
    WEIGHTS_MXFP4_MX_PLANES handles take)."""
    out = torch.empty_like(codes)
    for e in range(codes.shape[0]):
        tmt_moe.mxfp4_planes(codes[e], out[e])
    return out


def run_fp4(case, K, h, beta=0.0, Y0=None, fmt=tmt_moe.WEIGHTS_MXFP4, max_tokens=None):
    T, d = case["X"].shape
    E = case["W_up"].shape[0]
    qu, qd = mxfp4_experts(case["W_up"]), mxfp4_experts(case["W_down"])
    m = tmt_moe.MoE(max_tokens or max(T, 1), d, E, K, h, weight_format=fmt)
    Y = dev16(Y0) if Y0 is not None else torch.zeros(T, d, dtype=torch.bfloat16, device="cuda")
    bias = torch.from_numpy(case["bias"]).cuda() if case.get("bias") is not None else None
    cu, cd = dev8(qu["codes"]), dev8(qd["codes"])
    if fmt == tmt_moe.WEIGHTS_MXFP4_MX_PLANES:
        cu, cd = planes(cu), planes(cd)
    m.forward_mxfp4(dev16(case["X"]), dev16(case["Wr"]), cu, dev8(qu["scales"]),
                    cd, dev8(qd["scales"]), Y, beta=beta, bias=bias)
    out = {"Y": bf16_to_f32(Y.view(torch.int16).cpu().numpy().view(np.uint16))}
    out.update(m.routing())
    m.close()
    return out, qu["deq_bf16"], qd["deq_bf16"]


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("T,d,E,K,h", [
    (512, 1024, 32, 4, 256),   # the c5 router with a narrow expert
    (300, 256, 8, 2, 512),     # ragged T: partial row tiles in every expert segment
    (5, 512, 4, 2, 192),       # decode-sized batch, h not a multiple of the 256-column tile
    (100, 256, 1, 1, 128),     # one expert: no router, slot = token
    (1024, 256, 8, 2, 1024),   # a longer down GEMM (16 K steps) with partial row tiles
])
def test_mxfp4_against_oracle(orc, fmt, T, d, E, K, h):
    say(f"mxfp4 format {fmt} T={T} d={d} E={E} K={K} h={h}")
    case = make_case(T, d, E, K, h, seed=55 + T)
    Y0 = bf16_bits(np.random.default_rng(5).standard_normal((T, d)).astype(np.float32))
    g, wu, wd = run_fp4(case, K, h, beta=1.0, Y0=Y0, fmt=fmt)
    r = orc.forward(case["X"], case["Wr"], wu, wd, K, h, Y_in=Y0, beta=1.0)
    assert np.array_equal(g["idx"], r["idx"]) and np.array_equal(g["perm"], r["perm"])
    err = rel_l2(g["Y"], r["Y"])
    say(f"  Y rel-L2 {err:.2e}")
    assert err <= TOL


def test_mxfp4_mx_tracks_exact_format(orc):
    """The MX format differs from the exact-product format only by the
    activations' two-term MXFP6 rounding: well under the c5 tolerance."""
    T, d, E, K, h = 1024, 1024, 16, 4, 1024
    say(f"mxfp4 MX vs exact format T={T} d={d} E={E} K={K} h={h}")
    case = make_case(T, d, E, K, h, seed=77)
    ge, wu, wd = run_fp4(case, K, h, fmt=tmt_moe.WEIGHTS_MXFP4)
    gm, _, _ = run_fp4(case, K, h, fmt=tmt_moe.WEIGHTS_MXFP4_MX, max_tokens=4 * T)
    assert np.array_equal(ge["perm"], gm["perm"])
    d_mx = rel_l2(gm["Y"], ge["Y"])
    say(f"  MX vs exact rel-L2 {d_mx:.2e}")
    assert d_mx <= 5e-3


@pytest.mark.parametrize("fmt", FORMATS)
def test_mxfp4_c5_full_size(orc, fmt):
    cfg = CONFIGS["c5"]
    T, d, E, K, h = (cfg[k] for k in ("T", "d", "E", "K", "h"))
    say(f"c5 full size mxfp4 format {fmt} T={T} d={d} E={E} K={K} h={h}")
    case = make_case(T, d, E, K, h, with_dy=False)
    g, wu, wd = run_fp4(case, K, h, fmt=fmt)
    rr = orc.router(case["X"], case["Wr"], K)
    assert np.array_equal(g["idx"], rr["idx"])
    t = lambda a: torch.from_numpy(bf16_to_f32(a)).cuda()
    ref = moe_reference(t(case["X"]), t(case["Wr"]), t(wu), t(wd),
                        torch.from_numpy(rr["idx"].astype(np.int64)).cuda(), None, h,
                        need_grads=False)
    err = rel_l2(g["Y"], ref["Y"].cpu().numpy())
    say(f"  Y rel-L2 {err:.2e}")
    assert err <= TOL


@pytest.mark.parametrize("N,K", [(256, 1024), (1024, 4096), (192, 64), (64, 2112)])
def test_mxfp4_planes_layout(N, K):
    """tmt_moe_mxfp4_planes: plane p, row n holds bytes 32p .. 32p + 31 of
    code row n (columns 64p .. 64p + 63), against a numpy restatement."""
    say(f"mxfp4 planes layout N={N} K={K}")
    codes = np.random.default_rng(N + K).integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    out = torch.zeros(N * K // 2, dtype=torch.uint8, device="cuda")
    tmt_moe.mxfp4_planes(dev8(codes), out)
    torch.cuda.synchronize()
    want = codes.reshape(N, K // 64, 32).transpose(1, 0, 2)
    assert np.array_equal(out.cpu().numpy().reshape(K // 64, N, 32), want)


@pytest.mark.parametrize("T,d,E,K,h", [(300, 256, 8, 2, 512), (5, 512, 4, 2, 192), (2048, 1024, 32, 4, 256)])
def test_mx_planes_format_equals_mx(T, d, E, K, h):
    """Pre-packed weights run the same arithmetic as the MX format over the
    caller's layout: the outputs are bit-identical."""
    say(f"mx planes vs mx T={T} d={d} E={E} K={K} h={h}")
    case = make_case(T, d, E, K, h, seed=91 + T)
    a, _, _ = run_fp4(case, K, h, fmt=tmt_moe.WEIGHTS_MXFP4_MX)
    b, _, _ = run_fp4(case, K, h, fmt=tmt_moe.WEIGHTS_MXFP4_MX_PLANES)
    assert np.array_equal(a["Y"].view(np.uint32), b["Y"].view(np.uint32))


def test_mxfp4_handle_rejects_backward_and_bf16_forward():
    m = tmt_moe.MoE(16, 128, 4, 2, 128, weight_format=tmt_moe.WEIGHTS_MXFP4)
    X = torch.zeros(16, 128, dtype=torch.bfloat16, device="cuda")
    W = torch.zeros(4, 128, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(tmt_moe.MoeError, match="MXFP4"):
        m.forward(X, W[:, 0], W, W, X.clone())
    m.close()
