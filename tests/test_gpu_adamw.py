"""GPU parity of the multi-tensor AdamW (tmt_moe_adamw_*) against the
oracle, through the C ABI.

Bar: bit-exact. The squared gradient norm follows one fixed summation order
on both sides, and every float operation of the update is correctly rounded
on its own, so master weights, moments, the bf16 work copy and the norm must
match the oracle bit for bit, step after step.
"""
import sys

import numpy as np
import pytest
import torch

import tmt_moe
from synthetic import make_case

pytestmark = pytest.mark.gpu

B1, B2, EPS, WD = 0.9, 0.999, 1e-8, 0.01


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def host_params(rng, sizes_flags, work=True):
    ps = []
    for i, (n, fl) in enumerate(sizes_flags):
        ps.append(dict(master=rng.standard_normal(n).astype(np.float32),
                       m=(rng.uniform(-1, 1, n) * 0.01).astype(np.float32),
                       v=(np.abs(rng.uniform(-1, 1, n)) * 1e-4).astype(np.float32),
                       grad=rng.uniform(-1, 1, n).astype(np.float32),
                       work=np.zeros(n, np.uint16) if (work and i % 2 == 0) else None, flags=fl))
    return ps


def to_device(ps):
    out = []
    for q in ps:
        d = {k: torch.from_numpy(q[k].copy()).cuda() for k in ("master", "m", "v", "grad")}
        d["work"] = torch.from_numpy(q["work"].view(np.int16).copy()).cuda() if q["work"] is not None else None
        d["flags"] = q["flags"]
        out.append(d)
    return out


def assert_same(dev_ps, host_ps, what):
    for i, (d, h) in enumerate(zip(dev_ps, host_ps)):
        for k in ("master", "m", "v", "grad"):
            got = d[k].cpu().numpy()
            assert np.array_equal(got.view(np.uint32), h[k].view(np.uint32)), f"{what}: param {i} {k} differs"
        if h["work"] is not None:
            got = d["work"].cpu().numpy().view(np.uint16)
            assert np.array_equal(got, h["work"]), f"{what}: param {i} work differs"


SIZES = [(10000, 3), (8192 * 2 + 5, 3), (7, 3), (333, 1), (64, 0), (4096 * 3 + 1, 2), (8192, 3)]


def test_adamw_steps_bit_exact(orc):
    say("adamw: 3 steps with clipping, ragged sizes, flags, with and without work copies")
    rng = np.random.default_rng(1)
    hp = host_params(rng, SIZES)
    dp = to_device(hp)
    opt = tmt_moe.AdamW(dp)
    try:
        assert opt.chunks == sum((n + 8191) // 8192 for n, _ in SIZES)
        for step in (1, 2, 3):
            g = [rng.uniform(-1, 1, q["master"].size).astype(np.float32) for q in hp]
            for q, d, gg in zip(hp, dp, g):
                q["grad"][:] = gg
                d["grad"].copy_(torch.from_numpy(gg))
            lr, clip = 1e-3 * step, 0.05
            s_ref = orc.adamw_step(hp, clip, lr, B1, B2, EPS, WD, step)
            opt.step(step, lr, clip=clip, beta1=B1, beta2=B2, eps=EPS, weight_decay=WD)
            s = opt.sumsq()
            assert np.float64(s).view(np.uint64) == np.float64(s_ref).view(np.uint64), (s, s_ref)
            assert_same(dp, hp, f"step {step}")
    finally:
        opt.close()


def test_adamw_refuses_nonfinite_and_recovers(orc):
    say("adamw: non-finite gradient refuses the step; the next step runs")
    rng = np.random.default_rng(2)
    hp = host_params(rng, SIZES[:3])
    dp = to_device(hp)
    opt = tmt_moe.AdamW(dp)
    try:
        hp[1]["grad"][100] = np.inf
        dp[1]["grad"][100] = float("inf")
        s_ref = orc.adamw_step(hp, 1.0, 1e-3, B1, B2, EPS, WD, 1)
        opt.step(1, 1e-3, clip=1.0, beta1=B1, beta2=B2, eps=EPS, weight_decay=WD)
        assert not np.isfinite(opt.sumsq()) and not np.isfinite(s_ref)
        assert_same(dp, hp, "refused step")
        hp[1]["grad"][100] = 0.5
        dp[1]["grad"][100] = 0.5
        s_ref = orc.adamw_step(hp, 1.0, 1e-3, B1, B2, EPS, WD, 1)
        opt.step(1, 1e-3, clip=1.0, beta1=B1, beta2=B2, eps=EPS, weight_decay=WD)
        assert np.float64(opt.sumsq()).view(np.uint64) == np.float64(s_ref).view(np.uint64)
        assert_same(dp, hp, "step after the refused one")
        opt.zero_grads()
        torch.cuda.synchronize()
        for d in dp:
            assert torch.count_nonzero(d["grad"]).item() == 0
    finally:
        opt.close()


def test_adamw_on_block_gradients(orc):
    """The optimizer consuming what the block's backward wrote: fp32 dWr,
    dW_up and dW_down of a c1-shaped layer, updated in place; bf16 work
    copies are the next forward's weights."""
    say("adamw over the block's router and expert gradients (c1 shape)")
    T, d, E, K, h = 2048, 256, 4, 2, 1024
    case = make_case(T, d, E, K, h, seed=31)
    m = tmt_moe.MoE(T, d, E, K, h)
    try:
        dev16 = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)
        X, Wr, Wu, Wd, dY = (dev16(case[k]) for k in ("X", "Wr", "W_up", "W_down", "dY"))
        Y = torch.zeros(T, d, dtype=torch.bfloat16, device="cuda")
        m.forward(X, Wr, Wu, Wd, Y)
        dX = torch.empty_like(X)
        dWr = torch.empty(E, d, device="cuda")
        dWu = torch.empty(E, h, d, device="cuda")
        dWd = torch.empty(E, d, h, device="cuda")
        m.backward(dY, X, Wr, Wu, Wd, dX, dWr, dWu, dWd, 0.1, 1e-3)
        torch.cuda.synchronize()
    finally:
        m.close()
    rng = np.random.default_rng(5)
    grads = [dWr] + [dWu[e] for e in range(E)] + [dWd[e] for e in range(E)]
    hp, dp = [], []
    for g in grads:
        n = g.numel()
        q = dict(master=rng.standard_normal(n).astype(np.float32) * 0.02,
                 m=np.zeros(n, np.float32), v=np.zeros(n, np.float32),
                 grad=g.reshape(-1).cpu().numpy().copy(), work=np.zeros(n, np.uint16), flags=3)
        hp.append(q)
        dq = {k: torch.from_numpy(q[k].copy()).cuda() for k in ("master", "m", "v")}
        dq["grad"] = g.reshape(-1)
        dq["work"] = torch.zeros(n, dtype=torch.int16, device="cuda")
        dq["flags"] = 3
        dp.append(dq)
    opt = tmt_moe.AdamW(dp)
    try:
        s_ref = orc.adamw_step(hp, 1.0, 3e-4, B1, B2, EPS, WD, 1)
        opt.step(1, 3e-4, clip=1.0, beta1=B1, beta2=B2, eps=EPS, weight_decay=WD)
        assert np.float64(opt.sumsq()).view(np.uint64) == np.float64(s_ref).view(np.uint64)
        assert_same(dp, hp, "block gradients")
    finally:
        opt.close()


def test_adamw_c3_expert_set(orc):
    """A quarter of the c3 expert set (4 experts x 2 x 1024 x 4096 plus a
    16 x 1024 router): bit-exact after one clipped step."""
    say("adamw: 4 c3 experts (33.6M parameters), one step")
    rng = np.random.default_rng(6)
    sizes = [(16 * 1024, 3)] + [(4096 * 1024, 3)] * 8
    hp = host_params(rng, sizes)
    dp = to_device(hp)
    opt = tmt_moe.AdamW(dp)
    try:
        s_ref = orc.adamw_step(hp, 1.0, 1e-4, B1, B2, EPS, WD, 7)
        opt.step(7, 1e-4, clip=1.0, beta1=B1, beta2=B2, eps=EPS, weight_decay=WD)
        assert np.float64(opt.sumsq()).view(np.uint64) == np.float64(s_ref).view(np.uint64)
        assert_same(dp, hp, "c3 experts")
    finally:
        opt.close()
