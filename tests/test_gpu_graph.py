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
