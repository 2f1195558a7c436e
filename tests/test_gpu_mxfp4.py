"""GPU parity of the MXFP4 expert path (config c5) through the C ABI.

Reference: the same block with the exactly dequantised weights -- the CPU
oracle at a reduced token count and fp32 torch on the GPU at the full c5
size, with routing first matched bit for bit against the oracle router.
Tolerance 2e-2 relative L2 (the c5 contract)."""
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


def run_fp4(case, K, h, beta=0.0, Y0=None):
    T, d = case["X"].shape
    E = case["W_up"].shape[0]
    qu, qd = mxfp4_experts(case["W_up"]), mxfp4_experts(case["W_down"])
    m = tmt_moe.MoE(max(T, 1), d, E, K, h, weight_format=tmt_moe.WEIGHTS_MXFP4)
    Y = dev16(Y0) if Y0 is not None else torch.zeros(T, d, dtype=torch.bfloat16, device="cuda")
    bias = torch.from_numpy(case["bias"]).cuda() if case.get("bias") is not None else None
    m.forward_mxfp4(dev16(case["X"]), dev16(case["Wr"]), dev8(qu["codes"]), dev8(qu["scales"]),
                    dev8(qd["codes"]), dev8(qd["scales"]), Y, beta=beta, bias=bias)
    out = {"Y": bf16_to_f32(Y.view(torch.int16).cpu().numpy().view(np.uint16))}
    out.update(m.routing())
    m.close()
    return out, qu["deq_bf16"], qd["deq_bf16"]


def test_mxfp4_against_oracle(orc):
    T, d, E, K, h = 512, 1024, 32, 4, 256
    say(f"mxfp4 T={T} d={d} E={E} K={K} h={h}")
    case = make_case(T, d, E, K, h, seed=55)
    Y0 = bf16_bits(np.random.default_rng(5).standard_normal((T, d)).astype(np.float32))
    g, wu, wd = run_fp4(case, K, h, beta=1.0, Y0=Y0)
    r = orc.forward(case["X"], case["Wr"], wu, wd, K, h, Y_in=Y0, beta=1.0)
    assert np.array_equal(g["idx"], r["idx"]) and np.array_equal(g["perm"], r["perm"])
    err = rel_l2(g["Y"], r["Y"])
    say(f"  Y rel-L2 {err:.2e}")
    assert err <= TOL


def test_mxfp4_c5_full_size(orc):
    cfg = CONFIGS["c5"]
    T, d, E, K, h = (cfg[k] for k in ("T", "d", "E", "K", "h"))
    say(f"c5 full size mxfp4 T={T} d={d} E={E} K={K} h={h}")
    case = make_case(T, d, E, K, h, with_dy=False)
    g, wu, wd = run_fp4(case, K, h)
    rr = orc.router(case["X"], case["Wr"], K)
    assert np.array_equal(g["idx"], rr["idx"])
    t = lambda a: torch.from_numpy(bf16_to_f32(a)).cuda()
    ref = moe_reference(t(case["X"]), t(case["Wr"]), t(wu), t(wd),
                        torch.from_numpy(rr["idx"].astype(np.int64)).cuda(), None, h,
                        need_grads=False)
    err = rel_l2(g["Y"], ref["Y"].cpu().numpy())
    say(f"  Y rel-L2 {err:.2e}")
    assert err <= TOL


def test_mxfp4_handle_rejects_backward_and_bf16_forward():
    m = tmt_moe.MoE(16, 128, 4, 2, 128, weight_format=tmt_moe.WEIGHTS_MXFP4)
    X = torch.zeros(16, 128, dtype=torch.bfloat16, device="cuda")
    W = torch.zeros(4, 128, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(tmt_moe.MoeError, match="MXFP4"):
        m.forward(X, W[:, 0], W, W, X.clone())
    m.close()
