"""The C++ operator interface (include/tmt_moe.hpp) through the reference's
own layer tests, restated in tests/cpp/test_moe_layer.cpp: test_router
(tmt-cuda/src/architecture_test.cu:62-87), test_moe_backward (:228-264) and
the experts limit of tmt-cuda/tests/cli.sh:30-32. The binary is built by
__graft_entry__.build() (make -C tests/cpp)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")
BIN = os.path.join(CPP, "build", "test_moe_layer")
LIB = os.path.join(ROOT, "test-model-thing-cuda_amd", "libtmt_moe.so")


def _binary():
    if not os.path.exists(BIN) or os.path.getmtime(BIN) < os.path.getmtime(LIB):
        subprocess.run(["make", "-C", CPP], check=True, capture_output=True)
    return BIN


def test_cpp_layer_rejects_too_many_experts():
    """moe_keep_alloc with experts=65 prints the reason and exits(1), like the
    reference's CUDA_CHECK / config validation (no GPU call is reached)."""
    r = subprocess.run([_binary(), "reject"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1, r.stdout + r.stderr
    assert "moe_keep_alloc" in r.stdout and "experts=65" in r.stdout


@pytest.mark.gpu
def test_cpp_layer_reference_tests():
    r = subprocess.run([_binary()], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    for line in ("PASS MoE auxiliary and z-loss finite-difference gradients",
                 "PASS MoE backward: identical experts reproduce dense expert and input gradients",
                 "PASS MoE backward (up/SiLU/down experts)",
                 "PASS deferred router statistics", "ALL PASS"):
        assert line in r.stdout
