#!/usr/bin/env python3
"""Benchmark of the MI355X MoE block (BASELINE.json metric).

One step = forward + backward of the MoE feed-forward block on the c3
workload: T=32768 tokens, d=1024, E=16 experts, top-4, expert hidden h=4096,
bf16 with fp32 accumulation, router logits skewed by a Zipf(1.1) per-expert
bias (max expert load ~4x the mean), loss = <dY, Y> + 0.1*aux + 1e-3*z.
Inputs are synthetic (seed 1234) and resident in HBM before timing starts.

Prints one JSON line: tokens/s, ms/step, the fraction of bf16 MFMA peak of
the whole step, a per-kernel breakdown timed live with HIP events on the
launch stream, the roofline of the dominant kernel, decode latency at
T = 1/8/64 on the same weights, and the CPU oracle timed on this host's cores
on a bounded token slice of the same workload.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "test-model-thing-cuda_amd"))

METRIC = "MoE fwd+bwd tokens/s (E16 top4 d1024 bf16), % MFMA peak; decode µs/step"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
PEAK_FP4_TFLOPS = 10100.0   # MI355X dense MXFP4 MFMA


def kernel_work(phase, T, d, E, K, h):
    """Algorithmic work per launch: ('mfma', flops) or ('hbm', bytes)."""
    TK = T * K
    hn = h if h > 0 else d
    w = {
        "gemm_up": ("mfma", 2 * TK * d * hn),
        "gemm_down": ("mfma", 2 * TK * h * d),
        "gemm_dact": ("mfma", 2 * TK * d * h),
        "gemm_dw_down": ("mfma", 2 * TK * d * h),
        "gemm_dw_up": ("mfma", 2 * TK * hn * d),
        "gemm_dx": ("mfma", 2 * TK * hn * d),
        # X, Wr read; logits + probs, idx + gate, lse written
        "router": ("hbm", 2 * T * d + 2 * E * d + 8 * T * E + 8 * TK + 4 * T),
        # idx read; perm + slot_of written (plus block bases, negligible)
        "permute": ("hbm", 4 * TK + 8 * TK),
        "scan": ("hbm", 0),
        # expert outputs gathered, residual read + written, gates and slots
        "combine": ("hbm", 2 * TK * d + 4 * T * d + 8 * TK),
        # dY, X, expert outputs read; dO and X gathered to slot order written;
        # probs read, dlogits written; idx, gate, slot table; lse
        "combine_bwd": ("hbm", 4 * T * d + 6 * TK * d + 8 * T * E + 12 * TK + 4 * T),
        "router_dw": ("hbm", 2 * T * d + 4 * T * E + 4 * E * d),
        "scatter": ("hbm", 2 * TK * d + 2 * T * d + 4 * T * E + 4 * TK),
        # S read, H written, row mean + 1/std written, gamma + beta read
        "norm": ("hbm", 4 * T * d + 8 * T + 8 * d),
        # the router with the LayerNorm of its rows (routed batches of the
        # LayerNorm-fronted block): S read, H written, row statistics, gamma
        # and beta, then the router's own outputs
        "router_ln": ("hbm", 4 * T * d + 8 * T + 8 * d + 2 * E * d + 8 * T * E + 8 * TK + 4 * T),
        # scatter with the LayerNorm backward fused (d <= 2048): dXg rows, S,
        # dlogits, slots and row statistics read, dS written
        "scatter_ln": ("hbm", 2 * TK * d + 4 * T * d + 4 * T * E + 4 * TK + 8 * T),
    }
    return w.get(phase, ("hbm", 0))


def step_flops(T, d, E, K, h):
    fwd = 2 * T * d * E + (4 * T * K * d * h if h > 0 else 2 * T * K * d * d)
    bwd = 2 * (4 * T * K * d * h) + 4 * T * d * E if h > 0 else 2 * (2 * T * K * d * d) + 4 * T * d * E
    return fwd, bwd


def host_cpu():
    """CPU model (from /proc/cpuinfo), the thread count the OS reports
    (std::thread::hardware_concurrency / os.cpu_count) and the threads this
    process may run on (its affinity mask)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = os.cpu_count() or 1
    return model, os.cpu_count() or 1, allowed


# A GPU box grants one GPU's share of its host: 16 hardware threads, whatever
# the OS reports, so worker pools are capped there.
CPU_SHARE_THREADS = 16


def cpu_baseline(case, cfg, target_s=6.0, reps=3):
    """CPU oracle (test infrastructure) on a bounded token slice of the same
    workload, timed on this host's cores: one warm-up, then the median of
    `reps` timed runs (std::chrono-equivalent wall clock). Returns the
    cpu_baseline object."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import moe_oracle  # cpu_baseline leg only
    model, hw, allowed = host_cpu()
    threads = max(1, min(CPU_SHARE_THREADS, allowed))
    K, h = cfg["K"], cfg["h"]

    def run(ts):
        t0 = time.perf_counter()
        moe_oracle.backward(case["X"][:ts], case["Wr"], case["W_up"], case["W_down"], case["dY"][:ts],
                            K, h, bias=case.get("bias"), aux_coef=cfg.get("aux", 0.0),
                            z_coef=cfg.get("z", 0.0), threads=threads)
        return time.perf_counter() - t0

    # Two probes separate the per-call fixed cost (weight conversion, dW
    # buffers) from the per-token cost; the sample is sized for target_s per
    # run, and the first full-size run is the warm-up.
    t0 = run(64)
    t1 = run(512)
    per_tok = max((t1 - t0) / 448.0, 1e-6)
    ts = int(max(512, min(16384, 64 + (target_s - t0) / per_tok)))
    ts -= ts % 64
    run(ts)
    times = sorted(run(ts) for _ in range(reps))
    dt = times[len(times) // 2]
    return {"value": round(ts / dt, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu_model": model, "hardware_concurrency": hw, "affinity_threads": allowed,
            "runs_s": [round(t, 2) for t in times],
            "sample": f"oracle fwd+bwd (recomputes the forward) on the first {ts} tokens of the "
                      f"{cfg.get('name', 'c3')} workload with all {case['W_up'].shape[0]} experts, "
                      f"median of {reps} runs after one warm-up ({dt:.1f} s each), fp32 C++ on "
                      f"{threads} threads (this GPU's host share; the OS reports {hw} on a {model})"}


def bench_mxfp4(stream, reps=5):
    """c5: MXFP4 experts forward (T=65536, d=1024, E=32, top-4, h=4096) in
    both weight formats: "exact" (e2m1 weights expanded to bf16 in LDS, bf16
    MFMA) and "mx" (activations rounded to two MXFP6 terms, FP6 x FP4 scaled
    MFMA). Per-phase times come from the handle's own per-launch events."""
    import numpy as np
    import torch

    import tmt_moe
    from synthetic import CONFIGS, make_case, mxfp4_experts

    cfg = CONFIGS["c5"]
    T, d, E, K, h = (cfg[k] for k in ("T", "d", "E", "K", "h"))
    case = make_case(T, d, E, K, h, with_dy=False)
    qu, qd = mxfp4_experts(case["W_up"]), mxfp4_experts(case["W_down"])
    dev16 = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)
    dev8 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    X, Wr = dev16(case["X"]), dev16(case["Wr"])
    cu, su, cd, sd = dev8(qu["codes"]), dev8(qu["scales"]), dev8(qd["codes"]), dev8(qd["scales"])
    flops = 2 * T * d * E + 4 * T * K * d * h
    gemm_flops = 2 * T * K * d * h  # each expert GEMM

    def planes(codes):  # one-time packing, outside every timed region
        out = torch.empty_like(codes)
        for e in range(codes.shape[0]):
            tmt_moe.mxfp4_planes(codes[e], out[e])
        torch.cuda.synchronize()
        return out

    def run(fmt):
        Y = torch.zeros(T, d, dtype=torch.bfloat16, device="cuda")
        m = tmt_moe.MoE(T, d, E, K, h, weight_format=fmt)
        wu, wd = (planes(cu), planes(cd)) if fmt == tmt_moe.WEIGHTS_MXFP4_MX_PLANES else (cu, cd)
        fwd = lambda: m.forward_mxfp4(X, Wr, wu, su, wd, sd, Y, beta=0.0)
        for _ in range(2):
            fwd()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fwd()
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        m.set_profiling(True)
        m.profile(reset=True)
        for _ in range(reps):
            fwd()
        prof = m.profile(reset=True)
        m.set_profiling(False)
        m.close()
        # per forward (a phase may hold several launches)
        ph = {k: round(prof[k][0] / reps, 4) for k in ("router", "scan", "permute", "gemm_up", "gemm_down", "combine")}
        return ms, ph

    out = {"workload": f"c5: MXFP4 experts forward T={T} d={d} E={E} top-{K} h={h}"}
    for name, fmt in (("exact", tmt_moe.WEIGHTS_MXFP4), ("mx", tmt_moe.WEIGHTS_MXFP4_MX),
                      ("mx_planes", tmt_moe.WEIGHTS_MXFP4_MX_PLANES)):
        ms, ph = run(fmt)
        r = {"ms": round(ms, 4), "tokens_per_s": round(T / (ms / 1e3), 1),
             "tflops": round(flops / (ms / 1e3) / 1e12, 1), "phase_ms": ph}
        if name == "exact":
            # bf16 MFMA issue: the algorithmic flops once
            r["gemm_down_frac_bf16_peak"] = round(gemm_flops / (ph["gemm_down"] / 1e3) / 1e12 / PEAK_BF16_TFLOPS, 4)
            r["note"] = "weights streamed as e2m1+e8m0 and expanded to bf16 for bf16 MFMA"
        else:
            # FP6 x FP4 scaled MFMA issue (8 passes per 32x32x64, the FP4/FP6
            # rate): two activation terms, so twice the algorithmic flops
            r["gemm_down_frac_fp4_peak"] = round(2 * gemm_flops / (ph["gemm_down"] / 1e3) / 1e12 / PEAK_FP4_TFLOPS, 4)
            r["gemm_up_frac_fp4_peak"] = round(2 * gemm_flops / (ph["gemm_up"] / 1e3) / 1e12 / PEAK_FP4_TFLOPS, 4)
            r["note"] = ("activations as two MXFP6 terms (X rounded once per token into its K slots; SiLU(U) in "
                         "the up GEMM's epilogue), FP6 x FP4 v_mfma_scale_f32_32x32x64_f8f6f4; gemm_up includes the "
                         "quantise kernel" + (" (weights packed into K planes once, before timing)"
                                              if name == "mx_planes" else
                                              " and the per-call copy of both weight sets into K planes") +
                         "; frac counts both terms' MFMA flops against the 10.1 PF FP4/FP6 peak")
        out[name] = r
    out["faster"] = min(("exact", "mx", "mx_planes"), key=lambda k: out[k]["ms"])
    # headline fields keep their meaning: the faster format's numbers
    best = out[out["faster"]]
    out.update(ms=best["ms"], tokens_per_s=best["tokens_per_s"], tflops=best["tflops"],
               mfma_frac_fp4_peak=round(best["tflops"] / PEAK_FP4_TFLOPS, 4))
    return out


# The reference's own MoE benchmark (tmt-cuda/src/profile.cu:14-63): N=2048
# tokens, E=8, top-2, D=1280, single-linear experts (h = 0), backward with
# aux 0.01 and z 0.001; its FLOP model is fwd = 2NDE + 2NKD^2 and
# bwd = 2.2 x fwd (profile.cu:41-42, 60). The reference reports about 50% of
# its 49 TFLOP/s roof for this step (CHANGES.md:35, 46). The second shape is
# TMT's default width with a small MoE (config.h: dim 256, batch 8 x seqlen
# 128 tokens).
H0_SHAPES = {
    "reference_profile": dict(T=2048, d=1280, E=8, K=2, h=0, aux=0.01, z=0.001),
    "tmt_default_width": dict(T=1024, d=256, E=4, K=2, h=0, aux=0.01, z=0.001),
}


def bench_h0(name, steps=50, warmup=10):
    """fwd+bwd of the reference's expert shape (h = 0), timed with HIP events."""
    import numpy as np
    import torch

    import tmt_moe
    from synthetic import make_case

    cfg = H0_SHAPES[name]
    T, d, E, K = cfg["T"], cfg["d"], cfg["E"], cfg["K"]
    case = make_case(T, d, E, K, 0, seed=1234)
    dev16 = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)
    X, Wr, Wu, dY = (dev16(case[k]) for k in ("X", "Wr", "W_up", "dY"))
    Y = torch.zeros(T, d, dtype=torch.bfloat16, device="cuda")
    dX = torch.empty_like(X)
    dWr = torch.empty(E, d, device="cuda")
    dWu = torch.empty(E, d, d, device="cuda")
    m = tmt_moe.MoE(T, d, E, K, 0)
    try:
        def step():
            m.forward(X, Wr, Wu, None, Y, beta=1.0)
            m.backward(dY, X, Wr, Wu, None, dX, dWr, dWu, None, cfg["aux"], cfg["z"])

        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        # per-kernel breakdown from the handle's per-launch events (a separate
        # pass: the events add a little host time per launch)
        m.set_profiling(True)
        m.profile(reset=True)
        for _ in range(steps):
            step()
        prof = m.profile(reset=True)
        m.set_profiling(False)
    finally:
        m.close()
    phase_us = {k: round(v[0] / steps * 1e3, 2) for k, v in prof.items() if v[1] > 0}
    fwd = 2.0 * T * d * E + 2.0 * T * K * d * d
    flops = fwd * 3.2  # profile.cu's model: bwd = 2.2 x fwd
    tf = flops / (ms / 1e3) / 1e12
    return {"workload": f"{name}: fwd+bwd T={T} d={d} E={E} top-{K} h=0 (aux {cfg['aux']}, z {cfg['z']})",
            "ms_per_step": round(ms, 4), "tokens_per_s": round(T / (ms / 1e3), 1),
            "tflops_profile_model": round(tf, 2), "mfma_frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4),
            "phase_us": phase_us,
            "reference_published": "about 50% of a 49 TFLOP/s roof at N=2048 E=8 K=2 D=1280 "
                                   "(CHANGES.md:35,46), i.e. about 24.5 TFLOP/s, other hardware"}


COPY_PROBE_BYTES = 1 << 30


def copy_probe(reps=5):
    """Copies COPY_PROBE_BYTES between two device buffers `reps` times: a kernel
    whose HBM traffic is known (that many bytes read, that many written), so
    that FETCH_SIZE / WRITE_SIZE counters can be scaled to bytes."""
    import torch
    src = torch.ones(COPY_PROBE_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": COPY_PROBE_BYTES, "reps": reps}))


def source_digest():
    """SHA-256 (first 16 hex digits) of the kernel sources and the ABI
    header: the profiles under profiles/ record the digest of the code they
    measured, so numbers read from them can be matched to this tree."""
    import hashlib
    csrc = os.path.join(ROOT, "test-model-thing-cuda_amd", "csrc")
    files = sorted(os.path.join(csrc, f) for f in os.listdir(csrc)
                   if f.endswith((".hip", ".cpp", ".hpp")))
    files.append(os.path.join(ROOT, "include", "tmt_moe.h"))
    h = hashlib.sha256()
    for path in files:
        h.update(os.path.basename(path).encode())
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def measured_traffic(phase):
    """HBM bytes per launch of `phase` on c3, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (already scaled by the copy-probe factor).
    None when the summary does not list the kernel or was taken on other
    kernel sources than this tree's (its source_digest line differs)."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_c3.txt")
    digest, value = None, None
    try:
        with open(path) as f:
            for line in f:
                parts = line.split()
                if len(parts) >= 2 and parts[0] == "source_digest":
                    digest = parts[1]
                if len(parts) >= 4 and parts[0] == "traffic" and parts[1] == phase:
                    value = int(parts[2]) + int(parts[3])
    except OSError:
        return None
    return value if digest == source_digest() else None


def bench_decode(X, Wr, Wu, Wd, d, E, K, h, stream, reps=20, layers=8):
    """c4: decode forwards (beta = 1) at T = 1, 8, 64 tokens on c3-shaped layers.

    A step runs `layers` MoE layers, each with its own router and expert
    weights (layer 0 the c3 weights, the others fresh draws of the same
    distribution), so the experts stream from HBM as in a model: the experts
    one layer touches (67 to 268 MB) would otherwise stay in the 256 MB
    Infinity Cache across back-to-back calls of that one layer. µs per layer
    from HIP events around `reps` steps: launched eagerly, and with each step
    captured once as a HIP graph and replayed. The single-layer repeat of the
    earlier measurement is kept beside it ("same_layer_us")."""
    import math

    import numpy as np
    import torch

    import tmt_moe

    g = torch.Generator(device="cuda").manual_seed(11)
    nets = [(Wr, Wu, Wd)]
    for _ in range(layers - 1):
        nets.append(((torch.randn(E, d, device="cuda", generator=g) / math.sqrt(d)).to(torch.bfloat16),
                     (torch.randn(E, h, d, device="cuda", generator=g) / math.sqrt(d)).to(torch.bfloat16),
                     (torch.randn(E, d, h, device="cuda", generator=g) / math.sqrt(h)).to(torch.bfloat16)))
    out = {"layers": layers, "weights_per_layer_bytes": 2 * E * d * h * 2 + E * d * 2}
    md = tmt_moe.MoE(64, d, E, K, h)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn, n):
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / n

    for td in (1, 8, 64):
        Xd = X[:td].contiguous()
        Ys = [torch.zeros(td, d, dtype=torch.bfloat16, device="cuda") for _ in range(layers)]

        def step():
            for (wr, wu, wd), y in zip(nets, Ys):
                md.forward(Xd, wr, wu, wd, y, beta=1.0)

        # distinct experts per layer and the bytes they stream
        distinct = []
        for (wr, wu, wd), y in zip(nets, Ys):
            md.forward(Xd, wr, wu, wd, y, beta=1.0)
            distinct.append(int(np.unique(md.routing()["idx"]).size))
        for _ in range(3):
            step()
        us_layer = timed(step, reps) / layers
        # one step (all layers) captured as a HIP graph, replayed
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            step()
        stream.wait_stream(side)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph):
            step()
        for _ in range(3):
            graph.replay()
        us_graph = timed(graph.replay, reps) / layers
        # the earlier measurement: one layer called back to back
        wr, wu, wd = nets[0]
        one = lambda: md.forward(Xd, wr, wu, wd, Ys[0], beta=1.0)
        for _ in range(10):
            one()
        us_same = timed(one, 100)
        wbytes = float(np.mean(distinct)) * 2 * d * h * 2 + E * d * 2
        out[f"T{td}"] = {"us_per_layer": round(us_layer, 2), "us_per_layer_graph": round(us_graph, 2),
                         "same_layer_us": round(us_same, 2),
                         "distinct_experts_mean": round(float(np.mean(distinct)), 2),
                         "weight_bytes_mean": int(wbytes),
                         "hbm_gbs": round(wbytes / (us_layer * 1e-6) / 1e9, 1)}
        del graph
    md.close()
    del nets
    # The fixed cost of one hipGraphLaunch on this stack, from a graph of one
    # tiny kernel, beside the same kernel launched eagerly back to back: a
    # graph pays it once per replay, so a step of several layers amortises it.
    tiny = torch.zeros(256, device="cuda")
    gt = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        tiny.add_(1.0)
    stream.wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(gt):
        tiny.add_(1.0)
    for _ in range(5):
        gt.replay()
    out["graph_replay_floor_us"] = round(timed(gt.replay, 200), 2)
    out["eager_tiny_kernel_us"] = round(timed(lambda: tiny.add_(1.0), 200), 2)
    del gt
    torch.cuda.empty_cache()
    return out


def bench_layernorm(m, X, Wr, Wu, Wd, dY, T, d, E, K, h, aux_c, z_c, steps, warmup):
    """The LayerNorm-fronted block (tmt_moe_forward_ln + tmt_moe_backward_ln):
    ms per fwd+bwd step and the two LayerNorm phases' rates. S is the c3
    activation tensor, gamma ~ 1 + 0.1 N(0,1), beta ~ 0.1 N(0,1)."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(7)
    gamma = 1.0 + 0.1 * torch.randn(d, device="cuda", generator=g)
    beta = 0.1 * torch.randn(d, device="cuda", generator=g)
    hn = h if h > 0 else d
    Y = torch.zeros(T, d, dtype=torch.bfloat16, device="cuda")
    dS = torch.empty_like(X)
    dG, dB = torch.empty(d, device="cuda"), torch.empty(d, device="cuda")
    dWr = torch.empty(E, d, device="cuda")
    dWu = torch.empty(E, hn, d, device="cuda")
    dWd = torch.empty(E, d, h, device="cuda") if h > 0 else None

    def step():
        m.forward_ln(X, gamma, beta, Wr, Wu, Wd, Y, beta=1.0)
        m.backward_ln(dY, X, gamma, Wr, Wu, Wd, dS, dG, dB, dWr, dWu, dWd, aux_c, z_c)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    m.set_profiling(True)
    m.profile(reset=True)
    for _ in range(steps):
        step()
    prof = m.profile(reset=True)
    m.set_profiling(False)
    out = {"ms_per_step": round(ms, 4), "tokens_s": round(T / (ms / 1e3), 1)}
    # The router normalises its rows itself on routed batches that the VALU
    # router takes ("router" then carries the LayerNorm forward, and no
    # "norm" launch runs); where the matrix-core router applies, the
    # LayerNorm is its own "norm" launch and "router" is the plain router
    # over H. "scatter" carries the LayerNorm backward rows; "norm_bwd" is
    # the fixed-order dGamma/dBeta column sum of the per-workgroup partials.
    router_key = "router" if prof["norm"][1] > 0 else "router_ln"
    for ph, key in (("router", router_key), ("norm", "norm"), ("scatter", "scatter_ln"), ("norm_bwd", None)):
        tot, n = prof[ph]
        if n == 0:
            continue
        avg = tot / n
        k = {"avg_ms": round(avg, 4)}
        if key:
            _, work = kernel_work(key, T, d, E, K, h)
            k.update(gbs=round(work / avg / 1e6, 1), hbm_frac=round(work / avg / 1e6 / PEAK_HBM_GBS, 4))
        out[key or ph] = k
    return out


def bench_adamw(d, E, h, steps=10, warmup=2):
    """Multi-tensor AdamW (tmt_moe_adamw_step: gradient-norm pass + clipped
    update) over the block's parameters at this config: router [E, d] and
    E x (W_up [h, d] + W_down [d, h]), fp32 master / m / v / grad and a bf16
    work copy each. Algorithmic HBM bytes per element: 4 (norm pass reads
    grad) + 16 read + 14 written (update) = 34."""
    import torch
    import tmt_moe
    sizes = [E * d] + [h * d] * (2 * E)
    g = torch.Generator(device="cuda").manual_seed(3)
    params = []
    for n in sizes:
        params.append(dict(master=0.02 * torch.randn(n, device="cuda", generator=g),
                           m=torch.zeros(n, device="cuda"), v=torch.zeros(n, device="cuda"),
                           grad=1e-3 * torch.randn(n, device="cuda", generator=g),
                           work=torch.empty(n, dtype=torch.bfloat16, device="cuda"),
                           flags=tmt_moe.ADAMW_IN_NORM | tmt_moe.ADAMW_UPDATE))
    opt = tmt_moe.AdamW(params)
    try:
        for i in range(warmup):
            opt.step(i + 1, 1e-4, clip=1.0)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record(stream)
        for i in range(steps):
            opt.step(warmup + i + 1, 1e-4, clip=1.0)
        ev1.record(stream)
        torch.cuda.synchronize()
        ms = ev0.elapsed_time(ev1) / steps
        n = sum(sizes)
        gbs = 34 * n / (ms / 1e3) / 1e9
        return {"params": n, "chunks": opt.chunks, "ms_per_step": round(ms, 4),
                "gbs": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
                "bytes_per_param": 34, "finite": bool(opt.sumsq() == opt.sumsq())}
    finally:
        opt.close()
        del params
        torch.cuda.empty_cache()


def gemm_probe(reps=3):
    """For counter profiles: the c3 forward (router, grouped UP + DOWN,
    combine) `reps` times, then hipBLASLt (torch.matmul) on the dense
    equivalent of the DOWN GEMM -- all T*K routed rows against one expert's
    [d][h] weight, A[TK][h] . W^T -- `reps` times, random N(0,1) operands.
    Prints the hipBLASLt rate; the kernels' counters come from the profiler."""
    import numpy as np
    import torch

    import tmt_moe
    from synthetic import CONFIGS, make_case

    cfg = CONFIGS["c3"]
    T, d, E, K, h = (cfg[k] for k in ("T", "d", "E", "K", "h"))
    case = make_case(**cfg)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)
    X, Wr, Wu, Wd = (dev(case[k]) for k in ("X", "Wr", "W_up", "W_down"))
    bias = torch.from_numpy(case["bias"]).cuda() if case.get("bias") is not None else None
    Y = torch.zeros(T, d, dtype=torch.bfloat16, device="cuda")
    m = tmt_moe.MoE(T, d, E, K, h)
    for _ in range(reps):
        m.forward(X, Wr, Wu, Wd, Y, beta=0.0, bias=bias)
    m.close()
    g = torch.Generator(device="cuda").manual_seed(5)
    a = torch.randn(T * K, h, device="cuda", generator=g).to(torch.bfloat16)
    w = torch.randn(d, h, device="cuda", generator=g).to(torch.bfloat16)
    c = a @ w.t()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        c = a @ w.t()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    return {"hipblaslt_dense_down": {"shape": f"[{T * K}][{h}] x [{d}][{h}]^T", "ms": round(ms, 4),
                                     "tflops": round(2 * T * K * h * d / ms / 1e9, 1)}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c3")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-fp4", action="store_true", help="skip the c5 MXFP4 forward measurement")
    ap.add_argument("--no-ln", action="store_true",
                    help="skip the LayerNorm-fronted block measurement")
    ap.add_argument("--no-adamw", action="store_true",
                    help="skip the multi-tensor AdamW measurement")
    ap.add_argument("--adamw-only", action="store_true",
                    help="only the AdamW step over the config's block parameters")
    ap.add_argument("--no-profile", action="store_true",
                    help="time the step without per-kernel events")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a device copy of known size (HBM counter calibration)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the c4 decode measurement (T = 1, 8, 64 on the c3 weights)")
    ap.add_argument("--gemm-probe", action="store_true",
                    help="c3 forward GEMMs and hipBLASLt on the dense DOWN shape (for counter profiles)")
    ap.add_argument("--fp4-only", action="store_true",
                    help="only the c5 MXFP4 forward measurement (both weight formats)")
    ap.add_argument("--no-h0", action="store_true",
                    help="skip the reference-expert (h = 0) fwd+bwd measurements")
    ap.add_argument("--h0-only", action="store_true",
                    help="only the reference-expert (h = 0) fwd+bwd measurements, with per-kernel times")
    ap.add_argument("--source-digest", action="store_true",
                    help="print the digest of the kernel sources the profiles are tagged with")
    args = ap.parse_args()
    if args.source_digest:
        print(source_digest())
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    if args.copy_probe:
        copy_probe()
        return
    if args.gemm_probe:
        torch.cuda.set_device(0)
        print(json.dumps(gemm_probe()))
        return
    if args.fp4_only:
        torch.cuda.set_device(0)
        print(json.dumps(bench_mxfp4(torch.cuda.current_stream())))
        return
    if args.h0_only:
        torch.cuda.set_device(0)
        print(json.dumps({name: bench_h0(name) for name in H0_SHAPES}))
        return

    import tmt_moe
    from synthetic import CONFIGS, make_case

    cfg = CONFIGS[args.config]
    T, d, E, K, h = (cfg[k] for k in ("T", "d", "E", "K", "h"))
    hn = h if h > 0 else d
    torch.cuda.set_device(0)
    case = make_case(**cfg)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)
    X, Wr, Wu, dY = (dev(case[k]) for k in ("X", "Wr", "W_up", "dY"))
    Wd = dev(case["W_down"]) if h > 0 else None
    bias = torch.from_numpy(case["bias"]).cuda() if case.get("bias") is not None else None
    Y = torch.zeros(T, d, dtype=torch.bfloat16, device="cuda")
    dX = torch.empty_like(X)
    dWr = torch.empty(E, d, dtype=torch.float32, device="cuda")
    dWu = torch.empty(E, hn, d, dtype=torch.float32, device="cuda")
    dWd = torch.empty(E, d, h, dtype=torch.float32, device="cuda") if h > 0 else None
    aux_c, z_c = cfg.get("aux", 0.0), cfg.get("z", 0.0)
    if args.adamw_only:
        print(json.dumps({"adamw": bench_adamw(d, E, h if h > 0 else d, args.steps, args.warmup)}))
        return
    if args.decode_only:
        print(json.dumps({"decode": bench_decode(X, Wr, Wu, Wd, d, E, K, h, torch.cuda.current_stream())}))
        return
    m = tmt_moe.MoE(T, d, E, K, h)

    def step():
        m.forward(X, Wr, Wu, Wd, Y, beta=1.0, bias=bias)
        m.backward(dY, X, Wr, Wu, Wd, dX, dWr, dWu, dWd, aux_c, z_c)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # Headline: the timed steps run without per-kernel events.
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = ev0.elapsed_time(ev1) / args.steps
    aux, z, counts = m.stats()
    # Kernel table: a separate pass of the same step with HIP events around
    # every launch, on the launch stream.
    prof = {}
    prof_steps = max(args.steps // 2, 5)
    if not args.no_profile:
        m.set_profiling(True)
        m.profile(reset=True)
        for _ in range(prof_steps):
            step()
        prof = m.profile(reset=True)
        m.set_profiling(False)

    fwd_f, bwd_f = step_flops(T, d, E, K, h)
    kernels = {}
    for ph, (tot_ms, n) in prof.items():
        if n == 0:
            continue
        # the phase's work is done once per step, by all of its launches
        # (e.g. gemm_dx: the W_up transpose and the GEMM over it)
        per_step = tot_ms / prof_steps
        kind, work = kernel_work(ph, T, d, E, K, h)
        k = {"avg_ms": round(tot_ms / n, 4), "launches_per_step": n / prof_steps, "ms_per_step": round(per_step, 4),
             "share": round(per_step / ms_step, 4)}
        if kind == "mfma":
            k["tflops"] = round(work / per_step / 1e9, 1)
            k["mfma_frac"] = round(work / per_step / 1e9 / PEAK_BF16_TFLOPS, 4)
        elif work:
            k["gbs"] = round(work / per_step / 1e6, 1)
            k["hbm_frac"] = round(work / per_step / 1e6 / PEAK_HBM_GBS, 4)
        kernels[ph] = k
    roofline = None
    if kernels:
        dom = max(kernels, key=lambda p: kernels[p]["ms_per_step"])
        kind, work = kernel_work(dom, T, d, E, K, h)
        avg = kernels[dom]["ms_per_step"]
        if kind == "mfma":
            ach = work / avg / 1e9
            roofline = {"kernel": dom, "bound": "mfma", "achieved": round(ach, 1),
                        "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(ach / PEAK_BF16_TFLOPS, 4),
                        "traffic": measured_traffic(dom) if args.config == "c3" else None,
                        "work_per_launch": f"{work / 1e9:.1f} GFLOP = 2*T*K*d*h",
                        "timing": f"HIP events on the launch stream, {prof_steps} profiled steps "
                                  "after the headline steps",
                        "source_digest": source_digest()}
        else:
            ach = work / avg / 1e6
            roofline = {"kernel": dom, "bound": "hbm", "achieved": round(ach, 1),
                        "peak": PEAK_HBM_GBS, "unit": "GB/s",
                        "frac": round(ach / PEAK_HBM_GBS, 4),
                        "traffic": measured_traffic(dom) if args.config == "c3" else None,
                        "source_digest": source_digest()}

    ln = None
    if not args.no_ln:
        ln = bench_layernorm(m, X, Wr, Wu, Wd, dY, T, d, E, K, h, aux_c, z_c,
                             max(args.steps // 2, 1), 2)

    decode = None
    if not args.no_decode and args.config == "c3":
        decode = bench_decode(X, Wr, Wu, Wd, d, E, K, h, stream)

    adamw = None
    if not args.no_adamw:
        adamw = bench_adamw(d, E, h if h > 0 else d)

    fp4 = None
    if not args.no_fp4 and args.config == "c3":
        fp4 = bench_mxfp4(stream)

    h0 = None
    if not args.no_h0 and args.config == "c3":
        h0 = {name: bench_h0(name) for name in H0_SHAPES}

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(case, dict(cfg, name=args.config))

    tokens_s = T / (ms_step / 1e3)
    out = {
        "metric": METRIC,
        "value": round(tokens_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seed 1234, N(0,1) activations, N(0,1/sqrt(fan_in)) weights, Zipf(1.1) router bias)",
        "config": {"workload": f"{args.config}: MoE fwd+bwd T={T} d={d} E={E} top-{K} h={h}"
                               + (f" Zipf(1.1) skew {counts.max() / counts.mean():.2f}x" if E > 1 else ""),
                   "T": T, "d": d, "E": E, "K": K, "h": h, "aux": aux_c, "z": z_c,
                   "parallelism": "single GPU"},
        "mfma_frac_step": round((fwd_f + bwd_f) / (ms_step / 1e3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "step_tflop": round((fwd_f + bwd_f) / 1e12, 3),
        "wall_s_timed": round(wall, 3),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": kernels,
        "layernorm_block": ln,
        "adamw": adamw,
        "decode": decode,
        "mxfp4_forward": fp4,
        "reference_experts_h0": h0,
        "aux": round(aux, 6),
        "z": round(z, 6),
    }
    m.close()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
