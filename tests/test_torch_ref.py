"""Pins tests/torch_ref.py, the float reference of the full-size GPU parity
tests (c2/c3/c5), against the oracle at small shapes on the CPU.

* float64: moe_reference computes exactly the oracle's independent fp64 twin
  (orc_loss_f64, itself pinned by central finite differences in
  tests/test_oracle.py), so Y, the loss and every gradient agree to rounding
  noise (1e-10 relative L2). This covers the router softmax / top-k
  renormalisation, the aux and z-loss terms, the logit bias, up/down experts
  and the reference's single-linear experts (h = 0).
* float32: against the fp32 oracle, which rounds the expert activations to
  bf16 where the GPU does, the two differ only by that rounding (well inside
  the 1e-2 relative-L2 bar the full-size tests apply).
"""
import numpy as np
import pytest
import torch

from synthetic import bf16_to_f32, make_case
from torch_ref import moe_reference


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


CASES = [
    # T, d, E, K, h, with bias
    (96, 64, 6, 2, 128, True),
    (80, 64, 5, 3, 0, True),      # reference experts: one d x d linear, SiLU in combine
    (64, 128, 4, 2, 64, False),
    # the routing structures of the full-size GPU tests at small T and width
    (128, 128, 16, 4, 128, True),  # c2/c3: E = 16, top-4
    (96, 64, 32, 4, 64, False),    # c5: E = 32, top-4
    (40, 64, 1, 1, 64, False),     # dense: one expert, no router
    (48, 16, 4, 2, 0, True),       # TMT's own test width (architecture_test.cu:88-89)
    (36, 100, 8, 8, 72, True),     # widths off the 64 grid, top-8 of 8
]


def _inputs(T, d, E, K, h, with_bias, seed):
    case = make_case(T, d, E, K, h, seed=seed)
    if with_bias:
        case["bias"] = np.linspace(-0.5, 0.7, E).astype(np.float32)
    f = {k: bf16_to_f32(case[k]) for k in ("X", "Wr", "W_up", "dY")}
    f["W_down"] = bf16_to_f32(case["W_down"]) if h > 0 else None
    return case, f


@pytest.mark.parametrize("T,d,E,K,h,with_bias", CASES)
def test_torch_reference_equals_fp64_oracle(orc, T, d, E, K, h, with_bias):
    case, f = _inputs(T, d, E, K, h, with_bias, seed=11 + T)
    aux_c, z_c = 0.1, 1e-3
    o = orc.loss_f64(f["X"], f["Wr"], f["W_up"], f["W_down"] if h > 0 else np.zeros(1),
                     f["dY"], K, h, bias=case.get("bias"), aux_coef=aux_c, z_coef=z_c)
    t64 = lambda a: None if a is None else torch.from_numpy(np.asarray(a, np.float64))
    bias = t64(case.get("bias"))
    r = moe_reference(t64(f["X"]), t64(f["Wr"]), t64(f["W_up"]), t64(f["W_down"]),
                      torch.from_numpy(o["idx"].astype(np.int64)), t64(f["dY"]), h, bias=bias,
                      aux_coef=aux_c, z_coef=z_c)
    loss = float((t64(f["dY"]) * r["Y"]).sum()) + aux_c * r["aux"] + z_c * r["z"]
    assert abs(loss - o["loss"]) <= 1e-10 * max(1.0, abs(o["loss"]))
    # one expert: no router, so no router gradient
    names = ["dX", "dW_up"] + (["dWr"] if E > 1 else []) + (["dW_down"] if h > 0 else [])
    for n in names:
        err = rel_l2(r[n].numpy(), o[n])
        assert err <= 1e-10, f"{n}: torch fp64 reference vs oracle fp64 twin rel-L2 {err:.3e}"


@pytest.mark.parametrize("T,d,E,K,h,with_bias", CASES)
def test_torch_reference_fp32_tracks_fp32_oracle(orc, T, d, E, K, h, with_bias):
    case, f = _inputs(T, d, E, K, h, with_bias, seed=29 + T)
    aux_c, z_c = 0.1, 1e-3
    fw = orc.forward(case["X"], case["Wr"], case["W_up"], case["W_down"], K, h, bias=case.get("bias"))
    bw = orc.backward(case["X"], case["Wr"], case["W_up"], case["W_down"], case["dY"], K, h,
                      bias=case.get("bias"), aux_coef=aux_c, z_coef=z_c)
    t32 = lambda a: None if a is None else torch.from_numpy(np.asarray(a, np.float32))
    r = moe_reference(t32(f["X"]), t32(f["Wr"]), t32(f["W_up"]), t32(f["W_down"]),
                      torch.from_numpy(fw["idx"].astype(np.int64)), t32(f["dY"]), h,
                      bias=t32(case.get("bias")), aux_coef=aux_c, z_coef=z_c)
    assert abs(r["aux"] - fw["aux"]) <= 1e-5 * max(1.0, abs(fw["aux"]))
    assert abs(r["z"] - fw["z"]) <= 1e-5 * max(1.0, abs(fw["z"]))
    assert rel_l2(r["Y"].numpy(), fw["Y"]) <= 5e-3
    for n in ["dX", "dW_up"] + (["dWr"] if E > 1 else []) + (["dW_down"] if h > 0 else []):
        err = rel_l2(r[n].numpy(), bw[n])
        assert err <= 5e-3, f"{n}: rel-L2 {err:.3e}"
