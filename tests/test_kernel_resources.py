"""Every HIP kernel of the library compiles for gfx950 without scratch memory
and without VGPR spills.

Scratch in these kernels has come from register arrays indexed with a
runtime value (a loop with a runtime trip count over an accumulator array):
the array then lives in per-lane scratch, and every access becomes a memory
round trip (the router weight gradient ran 2x slower that way). The
compiler's resource-usage remarks report ScratchSize and VGPR spills per
kernel; this test compiles each source device-only, with the library's own
flags, and checks both are zero. CPU only: hipcc cross-compiles gfx950.
"""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "test-model-thing-cuda_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "--cuda-device-only", "-c", "-Rpass-analysis=kernel-resource-usage"]
SOURCES = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC) and shutil.which("hipcc") is None,
                                reason="hipcc not available")


def _remarks(src, out_dir):
    obj = os.path.join(out_dir, src + ".o")
    r = subprocess.run([HIPCC, *FLAGS, os.path.join(CSRC, src), "-o", obj],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    kernels, cur = {}, None
    for line in r.stderr.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            cur = m.group(1)
            kernels[cur] = {}
            continue
        m = re.search(r"remark:\s+(ScratchSize \[bytes/lane\]|VGPRs Spill): (\d+)", line)
        if m and cur is not None:
            kernels[cur][m.group(1)] = int(m.group(2))
    return kernels


@pytest.fixture(scope="module")
def resources():
    with tempfile.TemporaryDirectory() as d:
        procs = {}
        # compile the sources in parallel (gemm.hip dominates the time)
        from concurrent.futures import ThreadPoolExecutor
        with ThreadPoolExecutor(max_workers=min(len(SOURCES), max(1, (os.cpu_count() or 2) // 2))) as ex:
            futs = {src: ex.submit(_remarks, src, d) for src in SOURCES}
            for src, f in futs.items():
                procs[src] = f.result()
        return procs


@pytest.mark.parametrize("src", SOURCES)
def test_no_scratch_and_no_spills(resources, src):
    kernels = resources[src]
    assert kernels, f"no kernels reported for {src}"
    bad = {k: v for k, v in kernels.items()
           if v.get("ScratchSize [bytes/lane]", 0) > 0 or v.get("VGPRs Spill", 0) > 0}
    assert not bad, f"{src}: kernels with scratch or VGPR spills: {bad}"
