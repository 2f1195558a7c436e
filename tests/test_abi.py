"""C-ABI checks that need no GPU: the library loads, exports every function
include/tmt_moe.h declares, validates descriptors with clear errors, and the
product path has no route to the oracle or any CPU implementation."""
import ctypes
import os
import re

import pytest

import tmt_moe

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tmt_moe.h")
PKG = os.path.join(ROOT, "test-model-thing-cuda_amd")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tmt_moe_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = tmt_moe.load_library()
    names = declared_functions()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(tmt_moe.EXPORTED)


def test_workspace_size_matches_layout():
    c3 = tmt_moe.workspace_size(32768, 1024, 16, 4, 4096)
    TK = 32768 * 4
    # U, A, dU (TK x h) + O, dO, dXg, Xg (TK x d) + the LayerNorm output H
    # and its gradient (T x d) in bf16 dominate; the split-K tail adds one
    # 256 x 256 fp32 tile per CU (256 CUs on MI355X, the fallback without a GPU)
    # and GEMM_DX's transposed W_up one [E][d][h] bf16 copy
    big = (3 * TK * 4096 * 2 + 4 * TK * 1024 * 2 + 2 * 32768 * 1024 * 2 + 256 * 256 * 256 * 4
           + 16 * 1024 * 4096 * 2)
    assert big <= c3 <= big + (64 << 20)
    ref_mode = tmt_moe.workspace_size(2048, 256, 4, 2, 0)
    assert ref_mode < tmt_moe.workspace_size(2048, 256, 4, 2, 1024)


def test_shared_workspace_split():
    """The transient buffers (the reference's MoeWs) are reported apart from
    the per-layer state, so several layers can share one set: at c3 the
    backward operands dO, dU, dXg and Xg alone are 1.75 GiB."""
    total = tmt_moe.workspace_size(32768, 1024, 16, 4, 4096)
    layer, shared = tmt_moe.workspace_sizes(32768, 1024, 16, 4, 4096)
    assert layer + shared == total
    TK = 32768 * 4
    assert shared >= TK * 4096 * 2 + 3 * TK * 1024 * 2
    # per layer: U, SiLU(U) (TK x h) and O (TK x d) dominate
    assert 2 * TK * 4096 * 2 + TK * 1024 * 2 <= layer <= 2 * TK * 4096 * 2 + TK * 1024 * 2 + (128 << 20)
    # a forward-only MXFP4 handle keeps no backward buffers
    l4, s4 = tmt_moe.workspace_sizes(65536, 1024, 32, 4, 4096, tmt_moe.WEIGHTS_MXFP4)
    assert s4 < (64 << 20)


@pytest.mark.parametrize("desc,msg", [
    ((16, 0, 4, 2, 0), "d=0"),
    ((16, -3, 4, 2, 0), "d=-3"),
    ((16, 128, 0, 1, 0), "experts"),
    ((16, 128, 65, 1, 0), "experts"),
    ((16, 128, 4, 5, 0), "topk"),
    ((16, 128, 16, 9, 0), "topk"),
    ((16, 128, 4, 2, -64), "hidden"),
    ((0, 128, 4, 2, 0), "max_tokens"),
    # the MXFP4 formats keep whole 64-wide K steps (blocks of 32 along d and h)
    ((16, 100, 4, 2, 256, tmt_moe.WEIGHTS_MXFP4), "multiples of 64"),
    ((16, 256, 4, 2, 100, tmt_moe.WEIGHTS_MXFP4_MX), "multiples of 64"),
    ((16, 256, 4, 2, 100, tmt_moe.WEIGHTS_MXFP4_MX_PLANES), "multiples of 64"),
    ((16, 256, 4, 2, 256, 4), "weight_format"),
])
def test_invalid_descriptors_are_rejected(desc, msg):
    with pytest.raises(tmt_moe.MoeError) as ei:
        tmt_moe.workspace_size(*desc)
    assert ei.value.code == -1
    assert msg in str(ei.value)


@pytest.mark.parametrize("desc", [
    (14, 16, 1, 1, 0),      # TMT's small_config (architecture_test.cu:88-89): dense, dim 16
    (14, 16, 2, 2, 0),      # ... with two experts, top-2 (test_moe_backward)
    (64, 32, 4, 2, 0),      # tests/zig.sh:49 runs dim 32
    (1000, 100, 4, 2, 0),
    (1000, 100, 4, 2, 70),  # hidden not a multiple of 64 either
    (16, 1000, 16, 2, 0),
])
def test_any_width_is_accepted(desc):
    """TMT's validate_cfg takes any dim > 0 (tmt-cuda/src/config.h:46-52). The
    library runs such a layer on zero-padded internal copies of width
    ceil(d / 64) * 64 (and of hidden likewise), which the workspace holds."""
    T, d, E, K, h = desc
    size = tmt_moe.workspace_size(*desc)
    dp, hp = -(-d // 64) * 64, (-(-h // 64) * 64 if h else 0)
    assert size > tmt_moe.workspace_size(T, dp, E, K, hp)  # the padded copies come on top


@pytest.mark.parametrize("desc", [
    (16, 4096, 16, 4, 0),     # E*d = 65536: router weights beyond the LDS-staged size
    (16, 2560, 16, 4, 0),
    (16, 1280, 8, 2, 0),      # the reference's profile shape (tmt-cuda/src/profile.cu:17)
    (16, 2048, 64, 8, 512),   # widest router with up/down experts
])
def test_reference_dims_are_accepted(desc):
    """TMT accepts experts <= 16 with any dim (tmt-cuda/src/config.h:46-52);
    the library takes E up to 64 with any d."""
    assert tmt_moe.workspace_size(*desc) > 0


def test_layernorm_workspace_and_argument_checks():
    # chunk partials (512-row chunks) + level-1 sums (64 chunks per group), fp32
    nch = 32768 // 512
    assert tmt_moe.layernorm_workspace_size(32768, 1024) == (nch * 2 * 1024 + 1 * 2 * 1024) * 4
    assert tmt_moe.layernorm_workspace_size(0, 64) == (2 * 64 + 2 * 64) * 4
    # any width: partial rows of d rounded up to a multiple of 4
    assert tmt_moe.layernorm_workspace_size(16, 100) == (256 + 2 * 100) * 4
    with pytest.raises(tmt_moe.MoeError, match="d=0"):
        tmt_moe.layernorm_workspace_size(16, 0)
    lib = tmt_moe.load_library()
    f = ctypes.c_void_p
    # argument checks run before any device work
    assert lib.tmt_moe_layernorm_forward(None, 4, 0, None, None, None, None, None, None) == -1
    assert "d=0" in tmt_moe.last_error()
    assert lib.tmt_moe_layernorm_forward(None, 4, 128, None, None, None, None, None, None) == -1
    assert "non-NULL" in tmt_moe.last_error()
    fake = f(256)  # 256-byte aligned, never dereferenced: the size check fails first
    assert lib.tmt_moe_layernorm_backward(None, 4, 128, fake, fake, fake, fake, fake, fake, fake,
                                          fake, fake, ctypes.c_size_t(16)) == -1
    assert "smaller than" in tmt_moe.last_error()


def test_noalloc_layernorm_rejects_shapes_beyond_its_scratch():
    """tmt_moe_layernorm_backward_noalloc holds 4 MiB of device scratch: a
    shape whose workspace is larger fails its argument check, before any
    device call (so this runs without a GPU)."""
    lib = tmt_moe.load_library()
    T, d = 1 << 20, 2048
    assert tmt_moe.layernorm_workspace_size(T, d) > (4 << 20)
    p = ctypes.c_void_p(256)  # aligned stand-in: never dereferenced
    rc = lib.tmt_moe_layernorm_backward_noalloc(None, T, d, p, p, p, p, p, p, p, p)
    assert rc == -1
    assert b"bytes of scratch" in lib.tmt_moe_last_error()
    # the largest c3-sized standalone LayerNorm fits
    assert tmt_moe.layernorm_workspace_size(32768, 1024) <= (4 << 20)


def test_adamw_argument_checks():
    lib = tmt_moe.load_library()
    out = ctypes.c_void_p(0)
    assert lib.tmt_moe_adamw_create(None, -1, ctypes.byref(out)) == -1
    p = (tmt_moe.AdamwParam * 1)()
    p[0] = tmt_moe.AdamwParam(256, 512, 768, 1024 + 4, None, 10, 3)  # grad misaligned
    assert lib.tmt_moe_adamw_create(ctypes.cast(p, ctypes.c_void_p), 1, ctypes.byref(out)) == -1
    assert "16-byte aligned" in tmt_moe.last_error()
    p[0] = tmt_moe.AdamwParam(256, 512, 768, 1024, None, 10, 7)
    assert lib.tmt_moe_adamw_create(ctypes.cast(p, ctypes.c_void_p), 1, ctypes.byref(out)) == -1
    assert "flags" in tmt_moe.last_error()
    p[0] = tmt_moe.AdamwParam(256, 0, 768, 1024, None, 10, 3)
    assert lib.tmt_moe_adamw_create(ctypes.cast(p, ctypes.c_void_p), 1, ctypes.byref(out)) == -1
    assert "non-NULL" in tmt_moe.last_error()
    f = ctypes.c_float(0.0)
    assert lib.tmt_moe_adamw_step(None, None, f, f, f, f, f, f, 1) == -1
    assert lib.tmt_moe_adamw_zero_grads(None, None) == -1


def test_mxfp4_requires_hidden():
    with pytest.raises(tmt_moe.MoeError, match="hidden"):
        tmt_moe.workspace_size(16, 128, 4, 2, 0, tmt_moe.WEIGHTS_MXFP4)


def test_null_handle_is_an_error_not_a_crash():
    lib = tmt_moe.load_library()
    assert lib.tmt_moe_forward(None, None, 0, None, None, None, None, None, None,
                               ctypes.c_float(1.0)) == -1
    assert "NULL" in tmt_moe.last_error()
    assert lib.tmt_moe_destroy(None) == 0
    f = ctypes.c_float(0.0)
    assert lib.tmt_moe_forward_ln(None, None, 0, None, None, None, None, None, None, None,
                                  None, f) == -1
    assert lib.tmt_moe_backward_ln(None, None, None, None, None, None, None, None, f, f,
                                   None, None, None, None, None, None) == -1
    assert lib.tmt_moe_read_norm(None, None, None, None, None) == -1
    assert lib.tmt_moe_phase_name(0) == b"router"
    names = [lib.tmt_moe_phase_name(i) for i in range(tmt_moe.NPHASES)]
    assert all(names) and len(set(names)) == tmt_moe.NPHASES
    assert names[-2:] == [b"norm", b"norm_bwd"]
    assert lib.tmt_moe_phase_name(tmt_moe.NPHASES) == b"unknown"
    assert lib.tmt_moe_phase_name(99) == b"unknown"


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    monkeypatch.setattr(tmt_moe, "_lib", None)
    with pytest.raises(FileNotFoundError, match="no non-HIP implementation"):
        tmt_moe.load_library(str(tmp_path / "absent.so"))


def test_product_path_never_touches_the_oracle():
    for root in (PKG,):
        for dirpath, _, files in os.walk(root):
            for f in files:
                if f.endswith((".py", ".cpp", ".hip", ".hpp", ".h")):
                    text = open(os.path.join(dirpath, f)).read()
                    assert "moe_oracle" not in text and "liboracle" not in text, f
    # bench.py may use the oracle only inside its cpu_baseline leg
    import ast
    src = open(os.path.join(ROOT, "bench.py")).read()
    tree = ast.parse(src)
    allowed = [(n.lineno, n.end_lineno) for n in ast.walk(tree)
               if isinstance(n, ast.FunctionDef) and n.name == "cpu_baseline"]
    assert allowed, "bench.py must keep its oracle use inside cpu_baseline()"
    for node in ast.walk(tree):
        name = getattr(node, "id", None) or getattr(node, "name", None)
        if isinstance(node, ast.alias):
            name = node.name
        if name == "moe_oracle":
            line = getattr(node, "lineno", None)
            if line is None:  # alias nodes: find the import statement
                line = next(n.lineno for n in ast.walk(tree)
                            if isinstance(n, (ast.Import, ast.ImportFrom)) and node in n.names)
            assert any(a <= line <= b for a, b in allowed), f"bench.py:{line} uses the oracle"


@pytest.mark.parametrize("N,K,null,msg", [
    (100, 256, False, "multiples of 64"),
    (256, 96, False, "multiples of 64"),
    (0, 256, False, "multiples of 64"),
    (256, 256, True, "non-NULL"),
])
def test_mxfp4_planes_rejects_bad_arguments(N, K, null, msg):
    """The K-plane packer checks its arguments before any device work."""
    lib = tmt_moe.load_library()
    p = None if null else 4096
    rc = lib.tmt_moe_mxfp4_planes(None, p, N, K, p and 8192)
    assert rc != 0 and msg in tmt_moe.last_error()
