"""tmt_moe_layernorm_backward_noalloc against tmt_moe_layernorm_backward,
through the C ABI: the no-allocation variant runs the same kernels over the
library's own device scratch, so dS, dGamma and dBeta must be bit-identical
to the workspace variant. Two calls in a row, the second with a smaller
input (the scratch keeps the first call's contents). The rejection of
shapes whose workspace exceeds the scratch is a CPU test (test_abi.py)."""
import sys

import numpy as np
import pytest
import torch

import tmt_moe
from synthetic import bf16_bits

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _case(T, d, seed):
    rng = np.random.default_rng(seed)
    dev16 = lambda a: torch.from_numpy(bf16_bits(a).view(np.int16)).cuda().view(torch.bfloat16)
    S = dev16(rng.standard_normal((T, d)).astype(np.float32) * 2.0 + 0.5)
    dH = dev16(rng.standard_normal((T, d)).astype(np.float32))
    gamma = torch.from_numpy((1.0 + 0.2 * rng.standard_normal(d)).astype(np.float32)).cuda()
    beta = torch.from_numpy((0.1 * rng.standard_normal(d)).astype(np.float32)).cuda()
    H = torch.empty(T, d, dtype=torch.bfloat16, device="cuda")
    mean = torch.empty(T, device="cuda")
    rstd = torch.empty(T, device="cuda")
    tmt_moe.layernorm_forward(S, gamma, beta, H, mean, rstd)
    return S, dH, gamma, mean, rstd


def _outputs(T, d):
    nan = float("nan")
    return (torch.full((T, d), nan, dtype=torch.bfloat16, device="cuda"),
            torch.full((d,), nan, device="cuda"), torch.full((d,), nan, device="cuda"))


def test_noalloc_layernorm_backward_matches_workspace_variant():
    # each call smaller than the one before; the last at a width that is not a
    # multiple of 8 (element accesses)
    for T, d, seed in ((4096, 1024, 1), (777, 384, 2), (50, 100, 3)):
        say(f"no-alloc layernorm backward T={T} d={d}")
        S, dH, gamma, mean, rstd = _case(T, d, seed)
        ws = torch.empty(tmt_moe.layernorm_workspace_size(T, d) // 4 + 64, device="cuda")
        ref = _outputs(T, d)
        tmt_moe.layernorm_backward(S, dH, gamma, mean, rstd, *ref, ws)
        got = _outputs(T, d)
        tmt_moe.layernorm_backward_noalloc(S, dH, gamma, mean, rstd, *got)
        torch.cuda.synchronize()
        assert torch.equal(got[0].view(torch.int16), ref[0].view(torch.int16)), "dS differs"
        assert torch.equal(got[1].view(torch.int32), ref[1].view(torch.int32)), "dGamma differs"
        assert torch.equal(got[2].view(torch.int32), ref[2].view(torch.int32)), "dBeta differs"
        assert torch.isfinite(got[1]).all() and torch.isfinite(got[2]).all()


def test_noalloc_allocates_nothing_and_can_be_captured():
    """After a first call on the device (which looks the scratch's address up),
    a call leaves the device's free memory unchanged, and the call captured in
    a HIP graph replays to the workspace variant's results, bit for bit, with
    new inputs and eager work between the replays."""
    T, d = 1000, 512
    say(f"no-alloc free memory and graph capture T={T} d={d}")
    S, dH, gamma, mean, rstd = _case(T, d, 7)
    got = _outputs(T, d)
    tmt_moe.layernorm_backward_noalloc(S, dH, gamma, mean, rstd, *got)  # first call on the device
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    tmt_moe.layernorm_backward_noalloc(S, dH, gamma, mean, rstd, *got)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0, "the no-allocation call changed the device's free memory"

    ws = torch.empty(tmt_moe.layernorm_workspace_size(T, d) // 4 + 64, device="cuda")
    ref = _outputs(T, d)
    stream = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):  # warm-up on a side stream, as torch's graph capture expects
        tmt_moe.layernorm_backward_noalloc(S, dH, gamma, mean, rstd, *got)
    stream.wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        tmt_moe.layernorm_backward_noalloc(S, dH, gamma, mean, rstd, *got)
    rng = np.random.default_rng(11)
    for rep in range(3):
        dH.copy_(torch.from_numpy(bf16_bits(rng.standard_normal((T, d)).astype(np.float32)).view(np.int16))
                 .cuda().view(torch.bfloat16))
        for t in got:
            t.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        tmt_moe.layernorm_backward(S, dH, gamma, mean, rstd, *ref, ws)  # eager, between replays
        torch.cuda.synchronize()
        assert torch.equal(got[0].view(torch.int16), ref[0].view(torch.int16)), f"replay {rep}: dS differs"
        assert torch.equal(got[1].view(torch.int32), ref[1].view(torch.int32)), f"replay {rep}: dGamma differs"
        assert torch.equal(got[2].view(torch.int32), ref[2].view(torch.int32)), f"replay {rep}: dBeta differs"
