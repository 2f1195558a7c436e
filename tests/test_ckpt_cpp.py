"""The block's parameters in the reference's V3 checkpoint layout
(include/tmt_moe_ckpt.hpp), through tests/cpp/test_ckpt.cpp: FNV-1a known
answers, the trailer, corrupted and truncated files refused (host only), and
device round trips of both expert shapes with the bf16 work copies
regenerated (GPU). The binary is built by __graft_entry__.build()."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")
BIN = os.path.join(CPP, "build", "test_ckpt")
LIB = os.path.join(ROOT, "test-model-thing-cuda_amd", "libtmt_moe.so")


def _binary():
    if not os.path.exists(BIN) or os.path.getmtime(BIN) < os.path.getmtime(LIB):
        subprocess.run(["make", "-C", CPP], check=True, capture_output=True)
    return BIN


def test_checkpoint_format_host():
    r = subprocess.run([_binary(), "host"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "HOST PASS" in r.stdout


@pytest.mark.gpu
def test_checkpoint_round_trip_device():
    r = subprocess.run([_binary()], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    for line in ("PASS checkpoint round trip (reference-experts)",
                 "PASS checkpoint round trip (up-down-experts-with-layernorm)", "ALL PASS"):
        assert line in r.stdout
