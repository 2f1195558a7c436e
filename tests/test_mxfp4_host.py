"""MXFP4 host-side checks (no GPU): the product-side quantiser used for the
benchmark data equals the oracle's bit for bit, and the measured reason the
FP4 path keeps activations in bf16."""
import math

import numpy as np

import synthetic as sy


def test_numpy_quantiser_matches_oracle(orc):
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((96, 512)) / 20).astype(np.float32)
    w[0, :32] = 0.0                                       # all-zero block
    w[1, :7] = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]    # exact e2m1 midpoints
    w[1, 7] = 6.0                                         # sets the block scale to 2^0
    w[2, 3] = -0.0
    w[3, :32] = 1e30                                      # huge block
    w[4, :32] = 1e-30                                     # tiny block
    p1, s1 = sy.mxfp4_quantize(w)
    p2, s2 = orc.mxfp4_quantize(w)
    assert np.array_equal(p1, p2) and np.array_equal(s1, s2)
    assert np.array_equal(sy.mxfp4_dequantize(p1, s1), orc.mxfp4_dequantize(p2, s2, 512))


def test_expert_layout_round_trip():
    rng = np.random.default_rng(3)
    W = sy.bf16_bits((rng.standard_normal((3, 128, 256)) / 16).astype(np.float32))
    q = sy.mxfp4_experts(W)
    assert q["codes"].shape == (3, 128, 128) and q["scales"].shape == (3, 256 // 32, 128)
    deq = sy.bf16_to_f32(q["deq_bf16"])
    # dequantised MXFP4 values are exactly representable in bf16
    back = sy.mxfp4_dequantize(q["codes"], np.swapaxes(q["scales"], -1, -2))
    assert np.array_equal(deq, back)


def _e4m3(x):
    a = np.abs(x).astype(np.float64)
    e = np.maximum(np.floor(np.log2(np.maximum(a, 1e-300))), -6)
    step = 2.0 ** (e - 3)
    return (np.sign(x) * np.minimum(np.round(a / step) * step, 448.0)).astype(np.float32)


def _mxfp8(x):
    r, n = x.shape
    b = x.reshape(r, n // 32, 32)
    s = np.floor(np.log2(np.maximum(np.abs(b).max(-1, keepdims=True), 1e-30))) - 8
    return (_e4m3(b / 2.0 ** s) * 2.0 ** s).reshape(r, n).astype(np.float32)


def test_activation_precision_choice():
    """The gfx950 scaled MFMA needs both operands in an 8/6/4-bit format.
    Quantising the bf16 activations to MXFP8 (e4m3) costs more than the
    2e-2 rel-L2 budget against the dequantised fp32 result, while bf16
    activations times exactly dequantised weights stay far inside it, so the
    FP4 path expands weights to bf16 and runs bf16 MFMA."""
    rng = np.random.default_rng(0)
    T, d, h = 256, 512, 1024
    X = sy.bf16_to_f32(sy.bf16_bits(rng.standard_normal((T, d)).astype(np.float32)))
    Wu = (rng.standard_normal((h, d)) / math.sqrt(d)).astype(np.float32)
    Wd = (rng.standard_normal((d, h)) / math.sqrt(h)).astype(np.float32)
    Wuq = sy.mxfp4_dequantize(*sy.mxfp4_quantize(Wu))
    Wdq = sy.mxfp4_dequantize(*sy.mxfp4_quantize(Wd))
    silu = lambda u: u / (1 + np.exp(-u))
    bf = lambda a: sy.bf16_to_f32(sy.bf16_bits(a.astype(np.float32)))
    ref = silu(X @ Wuq.T) @ Wdq.T
    rel = lambda a: float(np.linalg.norm(a - ref) / np.linalg.norm(ref))
    bf16_path = rel(bf(silu(X @ Wuq.T)) @ Wdq.T)
    fp8_path = rel(_mxfp8(silu(_mxfp8(X) @ Wuq.T)) @ Wdq.T)
    assert bf16_path < 5e-3
    assert fp8_path > 2e-2
