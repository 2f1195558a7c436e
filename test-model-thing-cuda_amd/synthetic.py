"""Synthetic inputs for the MoE block (the BASELINE configurations).

All tensors are generated on the host with numpy's PCG64 from one seed
(1234 by default, the reference's config default, tmt-cuda/src/config.h:19)
and rounded to bf16 with round-to-nearest-even, so the GPU library and the
CPU oracle see bit-identical inputs.

  X, dY   ~ N(0, 1)                  (activations after LayerNorm)
  Wr      ~ N(0, 1/sqrt(d))          [E][d]
  W_up    ~ N(0, 1/sqrt(d))          [E][h][d]   ([E][d][d] when h == 0)
  W_down  ~ N(0, 1/sqrt(h))          [E][d][h]
  bias    Zipf profile -s*alpha*ln(e+1), alpha calibrated so that the most
          loaded expert receives `skew` times the mean load (c3).
"""
from __future__ import annotations

import numpy as np

CONFIGS = {
    # forward-only plumbing case (also run in full by the CPU oracle)
    "c1": dict(T=2048, d=256, E=4, K=2, h=1024, backward=False),
    # forward + backward, aux 0.1, z 1e-3
    "c2": dict(T=16384, d=512, E=8, K=2, h=2048, backward=True, aux=0.1, z=1e-3),
    # large model, Zipf(1.1)-skewed router, forward + backward
    "c3": dict(T=32768, d=1024, E=16, K=4, h=4096, backward=True, aux=0.1, z=1e-3,
               zipf=1.1, skew=4.0),
    # decode steps on the c3 weights
    "c4_t1": dict(T=1, d=1024, E=16, K=4, h=4096, backward=False),
    "c4_t8": dict(T=8, d=1024, E=16, K=4, h=4096, backward=False),
    "c4_t64": dict(T=64, d=1024, E=16, K=4, h=4096, backward=False),
    # MXFP4 experts, forward
    "c5": dict(T=65536, d=1024, E=32, K=4, h=4096, backward=False, mxfp4=True),
}


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# e2m1 rounding boundaries between consecutive codes 0..7 (magnitudes
# 0, .5, 1, 1.5, 2, 3, 4, 6); a value exactly on a boundary goes to the even code.
_E2M1_BOUNDS = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)


def mxfp4_quantize(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """OCP MXFP4 quantisation of fp32 rows (length a multiple of 32).

    Returns (codes [rows][n/2] uint8, low nibble = even element;
             scales [rows][n/32] uint8, e8m0). Scale exponent
    floor(log2(amax)) - 2 per block of 32, elements rounded to the nearest
    e2m1 value (ties to the even code), saturating at 6."""
    w = np.ascontiguousarray(w, np.float32)
    rows, n = w.reshape(-1, w.shape[-1]).shape
    blocks = w.reshape(rows, n // 32, 32)
    amax = np.abs(blocks).max(axis=2)
    _, ex = np.frexp(amax)                      # amax = f * 2^ex, f in [0.5, 1)
    se = np.where(amax > 0, np.clip(ex.astype(np.int32) - 3, -127, 127), 0)
    scaled = blocks * np.ldexp(np.float32(1.0), -se)[:, :, None].astype(np.float32)
    a = np.abs(scaled)
    code = np.zeros(a.shape, np.uint8)
    for k, b in enumerate(_E2M1_BOUNDS):
        code += ((a > b) if k % 2 == 0 else (a >= b)).astype(np.uint8)
    code |= np.signbit(scaled).astype(np.uint8) << 3
    code = code.reshape(rows, n)
    packed = (code[:, 0::2] | (code[:, 1::2] << 4)).astype(np.uint8)
    scales = (se + 127).astype(np.uint8)
    return packed.reshape(*w.shape[:-1], n // 2), scales.reshape(*w.shape[:-1], n // 32)


def mxfp4_dequantize(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Exact inverse of the code/scale encoding (fp32)."""
    grid = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6], np.float32)
    lo, hi = packed & 15, packed >> 4
    codes = np.stack([lo, hi], axis=-1).reshape(*packed.shape[:-1], packed.shape[-1] * 2)
    v = grid[codes]
    sc = np.ldexp(np.float32(1.0), scales.astype(np.int32) - 127).astype(np.float32)
    return v * np.repeat(sc, 32, axis=-1)


def _normal(rng: np.random.Generator, shape, std: float) -> np.ndarray:
    return bf16_bits(rng.standard_normal(shape, dtype=np.float32) * np.float32(std))


def zipf_bias(X: np.ndarray, Wr: np.ndarray, K: int, s: float = 1.1,
              skew: float = 4.0, sample: int = 8192) -> tuple[np.ndarray, float]:
    """Per-expert logit bias -s*alpha*ln(e+1) with alpha chosen by bisection so
    that max expert load / mean load ~= skew on (a sample of) the tokens."""
    E = Wr.shape[0]
    xs = bf16_to_f32(X[:sample])
    logits = xs @ bf16_to_f32(Wr).T
    prof = -s * np.log(np.arange(1, E + 1, dtype=np.float64))

    def ratio(alpha: float) -> float:
        l = logits + (alpha * prof)[None, :]
        top = np.argpartition(-l, K - 1, axis=1)[:, :K]
        cnt = np.bincount(top.ravel(), minlength=E)
        return cnt.max() / cnt.mean()

    lo, hi = 0.0, 8.0
    for _ in range(40):
        mid = 0.5 * (lo + hi)
        if ratio(mid) < skew:
            lo = mid
        else:
            hi = mid
    alpha = 0.5 * (lo + hi)
    return (alpha * prof).astype(np.float32), alpha


def mxfp4_experts(W: np.ndarray) -> dict:
    """Quantise bf16 expert weights [E][N][K] to the library's MXFP4 layout:
    codes [E][N][K/2] and block-major scales [E][K/32][N]; also returns the
    exactly dequantised weights as bf16 bits (the reference operand)."""
    packed, scales = mxfp4_quantize(bf16_to_f32(W))
    deq = mxfp4_dequantize(packed, scales)
    return {"codes": np.ascontiguousarray(packed),
            "scales": np.ascontiguousarray(np.swapaxes(scales, -1, -2)),
            "deq_bf16": bf16_bits(deq)}


def make_case(T: int, d: int, E: int, K: int, h: int, seed: int = 1234,
              zipf: float = 0.0, skew: float = 4.0, with_dy: bool = True,
              **_ignored) -> dict:
    """Host tensors (bf16 as uint16) for one configuration."""
    rng = np.random.Generator(np.random.PCG64(seed))
    hn = h if h > 0 else d
    case = {
        "X": _normal(rng, (T, d), 1.0),
        "Wr": _normal(rng, (E, d), 1.0 / np.sqrt(d)),
        "W_up": _normal(rng, (E, hn, d), 1.0 / np.sqrt(d)),
        "W_down": _normal(rng, (E, d, h), 1.0 / np.sqrt(h)) if h > 0 else None,
        "bias": None,
        "alpha": 0.0,
    }
    if with_dy:
        case["dY"] = _normal(rng, (T, d), 1.0)
    if zipf > 0 and E > 1:
        case["bias"], case["alpha"] = zipf_bias(case["X"], case["Wr"], K, zipf, skew)
    return case
