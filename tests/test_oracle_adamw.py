"""Pins the oracle's multi-tensor AdamW (orc_adamw_step) before it is used
as the GPU checker.

  * test_adamw_matches_reference_kat restates the reference's optimizer test
    (tmt-cuda/src/architecture_test.cu:404-434): random weights, moments and
    gradients, clipping exercised, double-precision expected values with the
    test's own tolerances, a parameter that must stay untouched, and a
    refused step on a non-finite gradient;
  * the canonical order of the squared gradient norm is restated
    independently in numpy (bit-equal) and checked against an exact sum;
  * flags and clip = 0 against closed forms.
"""
import math

import numpy as np
import pytest

B1, B2, EPS, WD = 0.9, 0.999, 1e-8, 0.01


def make_params(rng, sizes_flags):
    ps = []
    for n, fl in sizes_flags:
        ps.append(dict(master=rng.standard_normal(n).astype(np.float32),
                       m=(rng.uniform(-1, 1, n) * 0.01).astype(np.float32),
                       v=(np.abs(rng.uniform(-1, 1, n)) * 1e-4).astype(np.float32),
                       grad=rng.uniform(-1, 1, n).astype(np.float32),
                       work=np.zeros(n, np.uint16), flags=fl))
    return ps


def snapshot(ps):
    return [{k: (q[k].copy() if isinstance(q[k], np.ndarray) else q[k]) for k in q} for q in ps]


def bf16_rne(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def near(got, want, atol, rtol, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    bad = ~(np.abs(got - want) <= atol + rtol * np.abs(want))
    assert not bad.any(), f"{what}: {bad.sum()} mismatches, e.g. {got[bad][:3]} vs {want[bad][:3]}"


def test_adamw_matches_reference_kat(orc):
    rng = np.random.default_rng(9)
    # sizes: ragged, several chunks, tiny; index 3 is "stop" (in the norm, not
    # updated), index 4 is "tgt" (neither), as in the reference's model
    ps = make_params(rng, [(10000, 3), (8192 * 2 + 5, 3), (7, 3), (333, 1), (64, 0)])
    before = snapshot(ps)
    step0, clip, lr = 5, 0.05, 3e-4  # the reference test's 0-based step and gradclip
    s = orc.adamw_step(ps, clip, lr, B1, B2, EPS, WD, step0 + 1)
    sumsq = sum(math.fsum(np.asarray(q["grad"], np.float64) ** 2) for q in before if q["flags"] & 1)
    assert abs(s - sumsq) <= 1e-12 * sumsq
    scale = min(1.0, clip / max(math.sqrt(sumsq), 1e-12))
    assert scale < 1, "test does not exercise clipping"
    b1, b2 = float(np.float32(B1)), float(np.float32(B2))
    bc1 = float(np.float32(1.0) - np.float32(np.float32(B1) ** (step0 + 1)))
    bc2 = float(np.float32(1.0) - np.float32(np.float32(B2) ** (step0 + 1)))
    for q, q0 in zip(ps, before):
        if not q["flags"] & 2:
            for k in ("master", "m", "v"):
                assert np.array_equal(q[k], q0[k]), "parameter without the update flag changed"
            continue
        g = np.asarray(q0["grad"], np.float64) * scale
        nm = b1 * q0["m"] + (1 - b1) * g
        nv = b2 * q0["v"] + (1 - b2) * g * g
        nw = q0["master"] - lr * ((nm / bc1) / (np.sqrt(nv / bc2) + EPS) + WD * q0["master"])
        near(q["m"], nm, 1e-8, 1e-4, "first moment")
        near(q["v"], nv, 1e-10, 1e-4, "second moment")
        near(q["master"], nw, 1e-7, 1e-5, "weight")
        assert np.array_equal(q["work"], bf16_rne(q["master"])), "work copy is not bf16(master)"
    # non-finite gradient: the step is refused and nothing changes
    ps[1]["grad"][17] = np.nan
    keep = snapshot(ps)
    s2 = orc.adamw_step(ps, clip, lr, B1, B2, EPS, WD, step0 + 2)
    assert not math.isfinite(s2)
    for q, q0 in zip(ps, keep):
        for k in ("master", "m", "v", "work"):
            assert np.array_equal(q[k], q0[k], equal_nan=True), "refused step changed " + k


def numpy_canonical_sumsq(ps, waves_reversed=False):
    """Independent restatement of the GPU kernels' order: 8192-element
    chunks; thread t of 256 accumulates its 4-element groups t, t+256, ...
    in ascending element order; xor butterfly 32..1 per wave; waves added in
    order; then the chunk sums by the same scheme on 1024 threads (sixteen
    waves). waves_reversed plants a plausible mistake (the wave sums added
    from the last)."""
    lanes = np.arange(64)

    def block(t):
        w = []
        for wave in range(t.size // 64):
            l = t[wave * 64:(wave + 1) * 64].copy()
            for off in (32, 16, 8, 4, 2, 1):
                l = l + l[lanes ^ off]
            w.append(l[0])
        if waves_reversed:
            w = w[::-1]
        tot = w[0]
        for x in w[1:]:
            tot = tot + x
        return tot

    parts = []
    for q in ps:
        g = np.asarray(q["grad"], np.float64)
        for s in range(0, g.size, 8192):
            c = g[s:s + 8192]
            if not q["flags"] & 1:
                parts.append(0.0)
                continue
            acc = np.zeros(256)
            ngroups = (c.size + 3) // 4
            for gi in range(0, (ngroups + 255) // 256):
                for k in range(4):
                    idx = (gi * 256 + np.arange(256)) * 4 + k
                    ok = idx < c.size
                    acc = np.where(ok, acc + np.where(ok, c[np.minimum(idx, c.size - 1)], 0.0) ** 2, acc)
            parts.append(block(acc))
    parts = np.array(parts)
    t = np.zeros(1024)  # the final sum runs on one workgroup of 1024 threads
    for k0 in range(0, parts.size, 1024):
        chunk = parts[k0:k0 + 1024]
        t[:chunk.size] = t[:chunk.size] + chunk
    return block(t)


def test_adamw_norm_order_is_pinned(orc):
    rng = np.random.default_rng(3)
    sizes = [(8192 * 40 + 3, 3), (1, 1), (4097, 3), (300, 2), (8192 * 300, 1)]
    ps = make_params(rng, sizes)
    for q in ps:  # widely spread magnitudes make the order visible in the bits
        q["grad"] *= np.exp(rng.uniform(-12, 12, q["grad"].size)).astype(np.float32)
    want = numpy_canonical_sumsq(ps)
    exact = sum(math.fsum(np.asarray(q["grad"], np.float64) ** 2) for q in ps if q["flags"] & 1)
    got = orc.adamw_step(ps, 0.0, 0.0, B1, B2, EPS, 0.0, 1)
    assert np.float64(got).view(np.uint64) == np.float64(want).view(np.uint64)
    assert abs(got - exact) <= 1e-13 * exact
    # the bit-level comparison is sensitive: a plausible mistake in the order
    # (waves added from the last) gives different bits on this input
    wrong = numpy_canonical_sumsq(ps, waves_reversed=True)
    assert np.float64(wrong).view(np.uint64) != np.float64(got).view(np.uint64)


@pytest.mark.parametrize("clip", [0.0, 1e9])
def test_adamw_without_clipping_and_flags(orc, clip):
    rng = np.random.default_rng(4)
    ps = make_params(rng, [(1000, 3), (50, 2)])  # the second is updated but not in the norm
    before = snapshot(ps)
    lr, step = 1e-2, 1
    orc.adamw_step(ps, clip, lr, B1, B2, EPS, WD, step)
    b1, b2 = float(np.float32(B1)), float(np.float32(B2))
    bc1, bc2 = float(np.float32(1.0) - np.float32(B1)), float(np.float32(1.0) - np.float32(B2))
    for q, q0 in zip(ps, before):
        g = np.asarray(q0["grad"], np.float64)  # scale 1: no clipping
        nm = b1 * q0["m"] + (1 - b1) * g
        nv = b2 * q0["v"] + (1 - b2) * g * g
        nw = q0["master"] - lr * ((nm / bc1) / (np.sqrt(nv / bc2) + EPS) + WD * q0["master"])
        near(q["master"], nw, 1e-7, 1e-5, "weight")
