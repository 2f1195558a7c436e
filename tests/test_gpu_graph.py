"""Decode steps captured in a HIP graph and replayed equal eager steps.

A serving loop captures the decode step once and replays it, so the library's
forward must be capturable: no allocation, no host synchronisation and no
memset inside it, and state that lives across calls (the router's ticket for
T > 1) must come back to its start on every replay. Each case replays the
graph several times with new token inputs, with eager calls on the same
handle and host synchronisations between the replays, and checks every
replay bit for bit against an eager step on the same input.
"""
import sys

import numpy as np
import pytest
import torch

import tmt_moe
from synthetic import bf16_bits, make_case

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def dev(u16):
    return torch.from_numpy(np.ascontiguousarray(u16).view(np.int16)).cuda().view(torch.bfloat16)


@pytest.mark.parametrize("T,d,E,K,h", [
    (1, 256, 8, 2, 512),
    (8, 256, 16, 4, 512),
    (64, 128, 6, 3, 0),
    (5, 256, 1, 1, 256),
])
def test_decode_graph_replays_match_eager(T, d, E, K, h):
    say(f"graph replay T={T} d={d} E={E} K={K} h={h}")
    case = make_case(T, d, E, K, h, seed=31 + T)
    X = dev(case["X"])
    Wr = dev(case["Wr"])
    Wu = dev(case["W_up"])
    Wd = dev(case["W_down"]) if h > 0 else None
    m = tmt_moe.MoE(64, d, E, K, h)
    try:
        Yg = torch.zeros(T, d, dtype=torch.bfloat16, device="cuda")
        Ye = torch.zeros_like(Yg)
        stream = torch.cuda.current_stream()
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            m.forward(X, Wr, Wu, Wd, Yg, beta=0.0)
        stream.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            m.forward(X, Wr, Wu, Wd, Yg, beta=0.0)
        rng = np.random.default_rng(T)
        for rep in range(4):
            X.copy_(dev(bf16_bits(rng.standard_normal((T, d)).astype(np.float32))))
            Yg.zero_()
            graph.replay()
            torch.cuda.synchronize()
            routed = m.routing()
            m.forward(X, Wr, Wu, Wd, Ye, beta=0.0)
            torch.cuda.synchronize()
            again = m.routing()
            for key in ("idx", "perm", "offsets"):
                assert np.array_equal(routed[key], again[key]), f"replay {rep}: {key} differs"
            assert torch.equal(Yg, Ye), f"replay {rep}: Y differs from the eager step"
    finally:
        m.close()


@pytest.mark.parametrize("T,d,E,K,h", [
    (300, 256, 4, 2, 0),     # tiled GEMMs on 128 x 128 tiles (XCD runs)
    (200, 128, 6, 2, 256),
    (40, 128, 1, 1, 128),    # decode-sized forward, dense path
])
def test_training_step_graph_replays_match_eager(T, d, E, K, h):
    """Forward + backward captured in one graph (a training step under graph
    capture): every replay must equal an eager step bit for bit, outputs and
    gradients, with new inputs and eager steps between the replays."""
    say(f"graph replay fwd+bwd T={T} d={d} E={E} K={K} h={h}")
    case = make_case(T, d, E, K, h, seed=77 + T)
    X, Wr, Wu, dY = dev(case["X"]), dev(case["Wr"]), dev(case["W_up"]), dev(case["dY"])
    Wd = dev(case["W_down"]) if h > 0 else None
    hn = h if h > 0 else d
    m = tmt_moe.MoE(T, d, E, K, h)
    try:
        def buffers():
            return (torch.zeros(T, d, dtype=torch.bfloat16, device="cuda"),
                    torch.zeros(T, d, dtype=torch.bfloat16, device="cuda"),
                    torch.zeros(E, d, device="cuda"), torch.zeros(E, hn, d, device="cuda"),
                    torch.zeros(E, d, h, device="cuda") if h > 0 else None)

        def step(bufs):
            Y, dX, dWr, dWu, dWd = bufs
            m.forward(X, Wr, Wu, Wd, Y, beta=0.0)
            m.backward(dY, X, Wr, Wu, Wd, dX, dWr if E > 1 else None, dWu, dWd, 0.1, 1e-3)

        g, e = buffers(), buffers()
        stream = torch.cuda.current_stream()
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            step(g)
        stream.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step(g)
        rng = np.random.default_rng(T)
        for rep in range(3):
            X.copy_(dev(bf16_bits(rng.standard_normal((T, d)).astype(np.float32))))
            dY.copy_(dev(bf16_bits(rng.standard_normal((T, d)).astype(np.float32))))
            for t in g:
                if t is not None:
                    t.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            step(e)  # eager, between replays
            torch.cuda.synchronize()
            names = ("Y", "dX", "dWr", "dW_up", "dW_down")
            for name, a, b in zip(names, g, e):
                if a is None or (name == "dWr" and E == 1):
                    continue
                ia = a.view(torch.int16) if a.dtype == torch.bfloat16 else a.view(torch.int32)
                ib = b.view(torch.int16) if b.dtype == torch.bfloat16 else b.view(torch.int32)
                assert torch.equal(ia, ib), f"replay {rep}: {name} differs from the eager step"
    finally:
        m.close()
