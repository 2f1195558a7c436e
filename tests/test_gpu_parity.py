"""GPU parity: the HIP path, called through the C ABI, against the oracle.

Bars (from the build's contract):
  * routing -- router logits, top-k indices, expert offsets, permutation and
    slot table -- bit-exact against the CPU oracle;
  * floating-point outputs and gradients within 1e-2 relative L2 of the
    oracle's fp32 results (bf16 inputs, fp32 accumulation); at the full c2/c3
    sizes the fp32 reference is torch autograd on the GPU, fed with the
    routing that was just matched bit for bit.
Every test prints its case before touching the GPU.
"""
import sys

import numpy as np
import pytest
import torch

import tmt_moe
from synthetic import CONFIGS, bf16_bits, bf16_to_f32, make_case
from torch_ref import moe_reference

pytestmark = pytest.mark.gpu

REL_L2 = 1e-2  # north-star tolerance for floating outputs and gradients


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def dev(u16):
    return torch.from_numpy(np.ascontiguousarray(u16).view(np.int16)).cuda().view(torch.bfloat16)


def host_f32(t):
    return bf16_to_f32(t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16))


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def near(got, ref, atol, rtol, what):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    bad = ~(np.abs(got - ref) <= atol + rtol * np.abs(ref))
    assert not bad.any(), f"{what}: {bad.sum()} mismatches, e.g. {got[bad][:4]} vs {ref[bad][:4]}"


def run_gpu(case, K, h, beta=0.0, Y0=None, backward=False, aux=0.0, z=0.0, max_tokens=None,
            keep=False):
    T, d = case["X"].shape
    E = case["W_up"].shape[0]
    hn = h if h > 0 else d
    m = tmt_moe.MoE(max_tokens or max(T, 1), d, E, K, h)
    X = dev(case["X"])
    Wr = dev(case["Wr"])
    Wu = dev(case["W_up"])
    Wd = dev(case["W_down"]) if h > 0 else None
    bias = torch.from_numpy(case["bias"]).cuda() if case.get("bias") is not None else None
    Y = dev(Y0) if Y0 is not None else torch.zeros(T, d, dtype=torch.bfloat16, device="cuda")
    m.forward(X, Wr, Wu, Wd, Y, beta=beta, bias=bias)
    out = {"Y": host_f32(Y)}
    out.update(m.routing())
    out["aux"], out["z"], out["counts"] = m.stats()
    if backward:
        dY = dev(case["dY"])
        nan = float("nan")
        dX = torch.full((T, d), nan, dtype=torch.bfloat16, device="cuda")
        dWr = torch.full((E, d), nan, dtype=torch.float32, device="cuda")
        dWu = torch.full((E, hn, d), nan, dtype=torch.float32, device="cuda")
        dWd = torch.full((E, d, h), nan, dtype=torch.float32, device="cuda") if h > 0 else None
        m.backward(dY, X, Wr, Wu, Wd, dX, dWr if E > 1 else None, dWu, dWd, aux, z)
        torch.cuda.synchronize()
        out.update(dX=host_f32(dX), dW_up=dWu.cpu().numpy())
        out["dWr"] = dWr.cpu().numpy() if E > 1 else None
        out["dW_down"] = dWd.cpu().numpy() if h > 0 else None
    if keep:
        out["_moe"] = m
    else:
        m.close()
    return out


# Router logits of routed batches come from the matrix cores: the same exact
# bf16 products summed in another order, within a rounding bound of the
# oracle's canonical order; rows whose top-k ranking that bound could change
# are recomputed in the canonical order on the GPU, so the picks (and the
# offsets and permutation built from them) stay bit-exact.
LOGIT_ATOL, LOGIT_RTOL = 1e-4, 1e-5


def check_routing(g, r, E):
    assert np.array_equal(g["idx"], r["idx"]), "top-k indices differ"
    if E > 1:
        near(g["logits"], r["logits"], LOGIT_ATOL, LOGIT_RTOL, "logits")
        near(g["probs"], r["probs"], 1e-6, 1e-4, "probs")
    near(g["gate"], r["gate"], 1e-6, 1e-4, "gates")
    assert np.array_equal(g["offsets"], r["offsets"]), "expert offsets differ"
    assert np.array_equal(g["perm"], r["perm"]), "permutation differs"
    assert np.array_equal(g["slot_of"], r["slot_of"]), "slot table differs"


def check_grads(g, r, h, E):
    names = ["dX", "dW_up"] + (["dW_down"] if h > 0 else []) + (["dWr"] if E > 1 else [])
    for n in names:
        assert np.isfinite(g[n]).all(), f"{n} has unwritten/non-finite entries"
        err = rel_l2(g[n], r[n])
        say(f"  {n}: rel-L2 {err:.2e}")
        assert err <= REL_L2, f"{n} rel-L2 {err:.3e} > {REL_L2}"


def oracle_case(orc, case, K, h, Y0=None, beta=0.0, backward=False, aux=0.0, z=0.0):
    f = orc.forward(case["X"], case["Wr"], case["W_up"], case["W_down"], K, h,
                    bias=case.get("bias"), Y_in=Y0, beta=beta)
    if backward:
        f.update(orc.backward(case["X"], case["Wr"], case["W_up"], case["W_down"], case["dY"], K, h,
                              bias=case.get("bias"), aux_coef=aux, z_coef=z))
    return f


# ------------------------------------------------------------------ c1 ----

def test_c1_forward_against_oracle(orc):
    cfg = CONFIGS["c1"]
    say("c1 forward T=2048 d=256 E=4 K=2 h=1024 beta=1")
    case = make_case(**cfg)
    Y0 = bf16_bits(np.random.default_rng(1).standard_normal((cfg["T"], cfg["d"])).astype(np.float32))
    g = run_gpu(case, cfg["K"], cfg["h"], beta=1.0, Y0=Y0)
    r = oracle_case(orc, case, cfg["K"], cfg["h"], Y0=Y0, beta=1.0)
    check_routing(g, r, cfg["E"])
    err = rel_l2(g["Y"], r["Y"])
    say(f"  Y rel-L2 {err:.2e}")
    assert err <= REL_L2
    near(g["aux"], r["aux"], 1e-6, 1e-4, "aux")
    near(g["z"], r["z"], 1e-6, 1e-4, "z")
    assert np.array_equal(g["counts"], r["counts"])


def test_c1_backward_against_oracle(orc):
    cfg = CONFIGS["c1"]
    say("c1 forward+backward aux=0.1 z=1e-3")
    case = make_case(**cfg)
    g = run_gpu(case, cfg["K"], cfg["h"], backward=True, aux=0.1, z=1e-3)
    r = oracle_case(orc, case, cfg["K"], cfg["h"], backward=True, aux=0.1, z=1e-3)
    check_routing(g, r, cfg["E"])
    assert rel_l2(g["Y"], r["Y"]) <= REL_L2
    check_grads(g, r, cfg["h"], cfg["E"])


@pytest.mark.parametrize("T,d,E,K,h", [
    (1000, 256, 4, 2, 0),      # reference single-linear experts, SiLU in combine
    (777, 256, 1, 1, 0),       # reference dense path (experts=1, no router)
    (1237, 384, 8, 2, 256),    # ragged T, d not a multiple of 512
    (300, 512, 64, 8, 128),    # widest router (64 experts), top-8
    (500, 1024, 32, 4, 256),   # the c5 router shape
    (129, 128, 3, 3, 128),     # E == K, odd expert count
    (300, 64, 4, 2, 192),      # d = 64: one K = 64 tile in UP and DACT (the split ring's clamped reloads only)
    (333, 192, 5, 2, 320),     # d and h not multiples of the 256-wide GEMM tile
    (6, 256, 8, 2, 512),       # decode-sized: skinny expert GEMMs forward, tiled GEMMs backward
    (8, 1024, 16, 4, 4096),    # c3 weights at T = 8 (persistent skinny forward), forward + backward
    (211, 256, 12, 6, 256),    # top-6: the K = 6 combine / combine_bwd / scatter instantiations
    (97, 128, 7, 5, 128),      # top-5 over 7 experts, T below one router block
    (40, 256, 8, 2, 4096),     # decode DOWN in two K halves (combine forms O), then the backward reads O
    (24, 256, 8, 2, 4096),     # decode DOWN K halves with two row blocks (17..32 rows per expert)
    (20, 256, 8, 4, 4096),     # the same with top-4: the K = 4 partial combine
    (2048, 1280, 8, 2, 0),     # the reference's profile shape (tmt-cuda/src/profile.cu:17): h = 0, D = 1280
    (256, 2560, 16, 4, 0),     # E*d = 40960: router and dX scatter read Wr from memory, not LDS
    (96, 4096, 16, 4, 0),      # E*d = 65536, the widest TMT router (experts <= 16) at d = 4096
    (40, 2560, 16, 4, 0),      # decode-sized batch on the wide router
])
def test_shapes_against_oracle(orc, T, d, E, K, h):
    say(f"shape T={T} d={d} E={E} K={K} h={h} fwd+bwd")
    case = make_case(T, d, E, K, h, seed=T + d)
    aux, z = (0.1, 1e-3) if E > 1 else (0.0, 0.0)
    Y0 = bf16_bits(np.random.default_rng(T).standard_normal((T, d)).astype(np.float32))
    g = run_gpu(case, K, h, beta=1.0, Y0=Y0, backward=True, aux=aux, z=z)
    r = oracle_case(orc, case, K, h, Y0=Y0, beta=1.0, backward=True, aux=aux, z=z)
    check_routing(g, r, E)
    err = rel_l2(g["Y"], r["Y"])
    say(f"  Y rel-L2 {err:.2e}")
    assert err <= REL_L2
    check_grads(g, r, h, E)


@pytest.mark.parametrize("T,d,E,K,h", [
    (4, 1024, 16, 1, 256),     # fewer picks than experts: most of the expert-indexed grid is empty
    (16, 1024, 64, 2, 256),    # 64 experts: dispatch tables over every lane of the wave
    (33, 1024, 8, 2, 512),     # four 16-row blocks per expert
    (64, 2048, 16, 4, 256),    # the largest decode batch with 8-wave workgroups
    (12, 4096, 4, 2, 128),     # 16-wave workgroups, one 16-row block
    (20, 1024, 8, 8, 0),       # top-8 single-linear experts (no GEMM_DOWN; SiLU in the combine)
])
def test_decode_self_dispatch(orc, T, d, E, K, h):
    """Decode batches whose GEMM_UP completes the router's dispatch: the
    tables, the statistics and the block against the oracle, forward and
    backward."""
    say(f"decode self-dispatch T={T} d={d} E={E} K={K} h={h} fwd+bwd")
    case = make_case(T, d, E, K, h, seed=3 * T + E)
    Y0 = bf16_bits(np.random.default_rng(T + 1).standard_normal((T, d)).astype(np.float32))
    g = run_gpu(case, K, h, beta=1.0, Y0=Y0, backward=True, aux=0.1, z=1e-3)
    r = oracle_case(orc, case, K, h, Y0=Y0, beta=1.0, backward=True, aux=0.1, z=1e-3)
    check_routing(g, r, E)
    rr = orc.router(case["X"], case["Wr"], K, bias=case.get("bias"))
    rd = orc.dispatch(rr["idx"], E)
    assert np.array_equal(g["counts"], rd["counts"])
    aux, z = orc.aux_z(rr["probs"], rd["counts"], rr["lse"], K)
    near(g["aux"], aux, 1e-6, 1e-5, "aux")
    near(g["z"], z, 1e-6, 1e-5, "z")
    err = rel_l2(g["Y"], r["Y"])
    say(f"  Y rel-L2 {err:.2e}")
    assert err <= REL_L2
    check_grads(g, r, h, E)


def test_empty_batch():
    say("T=0 forward+backward")
    T, d, E, K, h = 0, 256, 4, 2, 256
    case = make_case(T, d, E, K, h)
    g = run_gpu(case, K, h, backward=True, aux=0.1, z=1e-3, max_tokens=16)
    assert g["aux"] == 0.0 and g["z"] == 0.0
    assert np.all(g["counts"] == 0) and np.all(g["offsets"] == 0)
    for n in ("dWr", "dW_up", "dW_down"):
        assert np.all(g[n] == 0.0), n


def test_dead_experts_get_zero_gradients(orc):
    say("dead experts: bias routes every token to experts 0 and 1")
    T, d, E, K, h = 640, 256, 8, 2, 256
    case = make_case(T, d, E, K, h, seed=5)
    case["bias"] = np.array([40, 40, -40, -40, -40, -40, -40, -40], np.float32)
    g = run_gpu(case, K, h, backward=True, aux=0.1, z=1e-3)
    r = oracle_case(orc, case, K, h, backward=True, aux=0.1, z=1e-3)
    check_routing(g, r, E)
    assert list(g["counts"]) == [T, T, 0, 0, 0, 0, 0, 0]
    assert np.all(g["dW_up"][2:] == 0.0) and np.all(g["dW_down"][2:] == 0.0)
    check_grads(g, r, h, E)


@pytest.mark.parametrize("T", [256, 8, 1])  # tiled router, decode router, single-token dispatch
def test_router_ties_go_to_lower_index(orc, T):
    say(f"router ties (T={T}): experts 2 and 4 have identical rows")
    d, E, K, h = 256, 6, 2, 128
    case = make_case(T, d, E, K, h, seed=6)
    case["Wr"][2] = case["Wr"][4]
    case["bias"] = np.array([-30, -30, 20, -30, 20, -30], np.float32)
    g = run_gpu(case, K, h)
    assert np.all(g["idx"] == np.array([2, 4]))
    assert np.array_equal(g["logits"][:, 2].view(np.uint32), g["logits"][:, 4].view(np.uint32))
    r = oracle_case(orc, case, K, h)
    check_routing(g, r, E)


@pytest.mark.parametrize("E,K", [(6, 2), (16, 4), (32, 8)])
def test_router_near_ties_follow_canonical_order(orc, E, K):
    """A batch large enough for the matrix-core router (T = 33000, at least
    one 128-row block per CU). Experts 1 and 3 (and 0 and 5) have weight rows
    one bf16 ulp apart in one element, so their logits differ by about 1e-4
    -- inside the matrix-core rounding bound: those rows must be ranked as
    the canonical order ranks them (the GPU recomputes them in that order),
    bit for bit."""
    T, d, h = 33000, 128, 0
    say(f"router near-ties E={E} K={K}")
    case = make_case(T, d, E, K, h, seed=61 + E)
    Wr = case["Wr"].copy()
    for a, b in ((1, 3), (0, 5)):
        Wr[b] = Wr[a]
        Wr[b, 7] = Wr[a, 7] + 1  # one ulp on the bf16 bit pattern
    case["Wr"] = Wr
    bias = np.full(E, -20.0, np.float32)
    bias[[0, 1, 3, 5]] = 20.0  # the near-tied pairs are the top picks
    case["bias"] = bias
    g = run_gpu(case, K, h)
    r = oracle_case(orc, case, K, h)
    check_routing(g, r, E)
    # The kernel's bound per row: delta = (4 (5d/64 + 24) 1.001 max_e A_e +
    # 8 (max |logit| + max |bias|)) 2^-24 with A_e = sum_k |x_k w_ek|; rows
    # with an adjacent gap above 2 delta among the top K + 1 keep the MFMA
    # logits. Where the oracle's gap is at most delta, the MFMA gap (within
    # 2 delta / 2.3 of it) is below 2 delta, so the GPU must have recomputed
    # the row canonically: its logits are the oracle's bits.
    x = np.abs(bf16_to_f32(case["X"]).astype(np.float64))
    w = np.abs(bf16_to_f32(case["Wr"]).astype(np.float64))
    A = (x @ w.T).max(axis=1)
    L = r["logits"].astype(np.float64)
    delta = (4 * (5 * d / 64 + 24) * 1.001 * A + 8 * (np.abs(L).max(axis=1) + np.abs(bias).max())) * 2.0 ** -24
    top = -np.sort(-L, axis=1)[:, :K + 1]
    certain = (np.diff(-top, axis=1) <= delta[:, None]).any(axis=1)
    say(f"  {certain.sum()} of {T} rows certain to be recomputed in the canonical order")
    assert certain.sum() > 100
    assert np.array_equal(g["logits"][certain].view(np.uint32), r["logits"][certain].view(np.uint32))


@pytest.mark.parametrize("T,d,E,K", [
    (40000, 1024, 16, 4),  # blocks walk two 128-row groups; the next group's chunks load during the epilogue
    (36000, 384, 8, 2),    # an odd number of 128-column chunks per row: the ring position flips between groups
    (33000, 1152, 32, 8),  # the widest rows whose Wr staging (32 rows) fits in LDS, 9 chunks per row
])
def test_matrix_core_router_group_walk(orc, T, d, E, K):
    """Batches with more 128-row groups than CUs: each block of the
    matrix-core router walks several groups, with Wr staged once and the
    X stream running on from one group into the next. Routing, offsets and
    the permutation bit-exact against the oracle router and dispatch at the
    full size; aux and z from the block statistics within float tolerance."""
    say(f"matrix-core router group walk T={T} d={d} E={E} K={K}")
    case = make_case(T, d, E, K, 0, seed=70 + E, with_dy=False)
    g = run_gpu(case, K, 0)
    rr = orc.router(case["X"], case["Wr"], K, bias=case.get("bias"))
    rd = orc.dispatch(rr["idx"], E)
    rr.update(rd)
    check_routing(g, rr, E)
    aux, z = orc.aux_z(rr["probs"], rd["counts"], rr["lse"], K)
    near(g["aux"], aux, 1e-6, 1e-4, "aux")
    near(g["z"], z, 1e-6, 1e-4, "z")


def test_runs_are_bitwise_deterministic():
    say("determinism: two identical fwd+bwd runs")
    T, d, E, K, h = 2000, 512, 8, 2, 512
    case = make_case(T, d, E, K, h, seed=8)
    a = run_gpu(case, K, h, backward=True, aux=0.1, z=1e-3)
    b = run_gpu(case, K, h, backward=True, aux=0.1, z=1e-3)
    for n in ("Y", "dX", "dWr", "dW_up", "dW_down", "perm", "logits"):
        assert np.array_equal(np.asarray(a[n]).view(np.uint32), np.asarray(b[n]).view(np.uint32)), n


# ------------------------------------------------------- c2 / c3 full size --

def _full_size(orc, name):
    cfg = CONFIGS[name]
    T, d, E, K, h = (cfg[k] for k in ("T", "d", "E", "K", "h"))
    say(f"{name} full size T={T} d={d} E={E} K={K} h={h} fwd+bwd")
    case = make_case(**cfg)
    g = run_gpu(case, K, h, backward=True, aux=cfg["aux"], z=cfg["z"])
    # routing against the oracle router + dispatch at full size
    rr = orc.router(case["X"], case["Wr"], K, bias=case.get("bias"))
    rd = orc.dispatch(rr["idx"], E)
    rr.update(rd)
    check_routing(g, rr, E)
    aux, z = orc.aux_z(rr["probs"], rd["counts"], rr["lse"], K)
    near(g["aux"], aux, 1e-6, 1e-4, "aux")
    near(g["z"], z, 1e-6, 1e-4, "z")
    # floating outputs against fp32 torch autograd on the matched routing
    t = lambda a: torch.from_numpy(bf16_to_f32(a)).cuda()
    ref = moe_reference(t(case["X"]), t(case["Wr"]), t(case["W_up"]),
                        t(case["W_down"]), torch.from_numpy(rr["idx"].astype(np.int64)).cuda(),
                        t(case["dY"]), h,
                        bias=None if case.get("bias") is None else torch.from_numpy(case["bias"]).cuda(),
                        aux_coef=cfg["aux"], z_coef=cfg["z"])
    err = rel_l2(g["Y"], ref["Y"].cpu().numpy())
    say(f"  Y rel-L2 {err:.2e}")
    assert err <= REL_L2
    refn = {k: (v.cpu().numpy() if torch.is_tensor(v) else v) for k, v in ref.items()}
    check_grads(g, refn, h, E)
    return g, case


def test_c2_full_size(orc):
    _full_size(orc, "c2")


def test_c3_full_size_zipf(orc):
    g, case = _full_size(orc, "c3")
    cnt = g["counts"]
    skew = cnt.max() / cnt.mean()
    say(f"  c3 load skew max/mean = {skew:.2f} (alpha {case['alpha']:.3f})")
    assert 3.0 < skew < 5.0


@pytest.mark.parametrize("T", [1, 8, 64])
def test_decode_steps_against_oracle(orc, T):
    cfg = CONFIGS["c3"]
    say(f"decode T={T} on c3 weights")
    case = make_case(T, cfg["d"], cfg["E"], cfg["K"], cfg["h"], seed=1234 + T)
    Y0 = bf16_bits(np.random.default_rng(T).standard_normal((T, cfg["d"])).astype(np.float32))
    g = run_gpu(case, cfg["K"], cfg["h"], beta=1.0, Y0=Y0, max_tokens=64)
    r = oracle_case(orc, case, cfg["K"], cfg["h"], Y0=Y0, beta=1.0)
    check_routing(g, r, cfg["E"])
    assert rel_l2(g["Y"], r["Y"]) <= REL_L2


@pytest.mark.parametrize("T,d,E,K,h", [
    (1, 192, 5, 2, 320),     # one token, d and h not multiples of 256
    (3, 256, 4, 2, 0),       # reference single-linear experts
    (17, 128, 3, 3, 128),    # two 16-row blocks per expert, E == K
    (40, 512, 64, 8, 128),   # widest router, top-8, up to 40 rows per expert
    (64, 256, 1, 1, 0),      # dense path at the decode-kernel limit
    (65, 192, 5, 2, 320),    # first token count on the tiled path
    (9, 128, 4, 2, 1088),    # down-projection K of 17 x 64: one tile per workgroup
    (33, 256, 8, 2, 2048),   # three 16-row blocks, 8 waves of 256-element chunks
    (2, 128, 64, 8, 256),    # 64 experts, 16 ranks of one row, one 64-element unit per wave
    (7, 320, 6, 3, 768),     # 20 column tiles of DOWN, a single row block per expert
    (1, 64, 2, 1, 256),      # a single token and expert, d of one unit
    (24, 1024, 8, 2, 4096),  # persistent UP, two resident row blocks, 2-3 tiles per workgroup
    (12, 512, 3, 2, 2048),   # persistent DOWN over 8 waves, one tile and a past-the-end prefetch
    (1, 256, 8, 1, 1024),    # one token: down GEMM + combine in one launch, top-1, 4 waves
    (1, 512, 16, 8, 2048),   # one token, top-8 (32 rows per workgroup), 8 waves
    (1, 1024, 64, 4, 4096),  # one token, 64 experts, 16 waves
])
def test_decode_shapes_against_oracle(orc, T, d, E, K, h):
    """Decode-sized batches (T <= 64 use the weight-streaming expert GEMMs);
    the backward reads the U / SiLU(U) / O those kernels wrote."""
    say(f"decode shape T={T} d={d} E={E} K={K} h={h} fwd+bwd")
    case = make_case(T, d, E, K, h, seed=7 * T + d)
    aux, z = (0.1, 1e-3) if E > 1 else (0.0, 0.0)
    Y0 = bf16_bits(np.random.default_rng(T + 1).standard_normal((T, d)).astype(np.float32))
    g = run_gpu(case, K, h, beta=1.0, Y0=Y0, backward=True, aux=aux, z=z, max_tokens=128)
    r = oracle_case(orc, case, K, h, Y0=Y0, beta=1.0, backward=True, aux=aux, z=z)
    check_routing(g, r, E)
    err = rel_l2(g["Y"], r["Y"])
    say(f"  Y rel-L2 {err:.2e}")
    assert err <= REL_L2
    check_grads(g, r, h, E)


@pytest.mark.parametrize("E,K", [(64, 8), (16, 4), (3, 3)])
def test_single_token_dispatch_with_bias(orc, E, K):
    """T = 1 finishes the dispatch in the router's registers (ballots over
    the picked lanes); a Zipf logit bias, every expert count from 1 to 64
    lanes, K up to E."""
    say(f"single token E={E} K={K} with a Zipf logit bias, fwd+bwd")
    d, h = 256, 256
    case = make_case(1, d, E, K, h, seed=100 + E, zipf=1.1)
    Y0 = bf16_bits(np.random.default_rng(E).standard_normal((1, d)).astype(np.float32))
    g = run_gpu(case, K, h, beta=1.0, Y0=Y0, backward=True, aux=0.1, z=1e-3, max_tokens=4)
    r = oracle_case(orc, case, K, h, Y0=Y0, beta=1.0, backward=True, aux=0.1, z=1e-3)
    check_routing(g, r, E)
    near(g["aux"], r["aux"], 1e-6, 1e-4, "aux")
    near(g["z"], r["z"], 1e-6, 1e-4, "z")
    assert list(g["counts"]) == [int(e in r["idx"][0]) for e in range(E)]
    assert rel_l2(g["Y"], r["Y"]) <= REL_L2
    check_grads(g, r, h, E)


def test_decode_all_tokens_on_two_experts(orc):
    """T = 64 with every token routed to experts 0 and 1: 64 rows per expert,
    the largest row count the decode kernel handles."""
    say("decode T=64, bias routes every token to experts 0 and 1")
    T, d, E, K, h = 64, 256, 8, 2, 256
    case = make_case(T, d, E, K, h, seed=11)
    case["bias"] = np.array([40, 40, -40, -40, -40, -40, -40, -40], np.float32)
    g = run_gpu(case, K, h, backward=True, aux=0.1, z=1e-3)
    r = oracle_case(orc, case, K, h, backward=True, aux=0.1, z=1e-3)
    check_routing(g, r, E)
    assert list(g["counts"]) == [T, T, 0, 0, 0, 0, 0, 0]
    assert rel_l2(g["Y"], r["Y"]) <= REL_L2
    check_grads(g, r, h, E)
