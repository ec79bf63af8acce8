"""Register budget of the matrix-core attention kernels (CPU: compiles the device code only).

The packed loop is tuned to three waves per SIMD: a change that adds live
registers can make the compiler spill to scratch, which slows the kernel by
a large factor while every parity test still passes. This test compiles
tt_attn.hip for gfx950 with the resource remarks and checks, per kernel
instantiation, the VGPR count, the scratch size and the occupancy.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "tritiercache_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# No group size spills (eight-head groups are held to 168 VGPRs).
LIMITS = {1: 0, 2: 0, 4: 0, 8: 0}


@pytest.fixture(scope="module")
def resources(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("res") / "tt_attn.o"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Xclang",
           "-target-feature", "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form=1",
           "--cuda-device-only", "-c", "-o", str(out), "-Rpass-analysis=kernel-resource-usage",
           os.path.join(CSRC, "tt_attn.hip")]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    kernels = {}
    name = None
    for line in r.stderr.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            kernels[name] = {}
            continue
        m = re.search(r"remark:\s+(VGPRs|ScratchSize \[bytes/lane\]|Occupancy \[waves/SIMD\]): (\d+)", line)
        if m and name:
            kernels[name][m.group(1).split(" ")[0]] = int(m.group(2))
    return kernels


@pytest.mark.parametrize("kernel", ["attn_packed_kernel", "attn_batched_kernel"])
@pytest.mark.parametrize("gp", [1, 2, 4, 8])
def test_no_spills_three_waves(resources, kernel, gp):
    found = {k: v for k, v in resources.items() if re.search(rf"{kernel}ILi{gp}E", k)}
    # fp32 and fp16 metadata, and for the single-sequence kernel with 2, 4 or 8
    # heads per group also the paired head_dim-64 variants of both
    paired = kernel == "attn_packed_kernel" and gp in (2, 4, 8)
    assert len(found) == (4 if paired else 2), (kernel, gp, sorted(found))
    for name, res in found.items():
        assert res["ScratchSize"] <= LIMITS[gp], (name, res)
        assert res["VGPRs"] <= 168, (name, res)
        assert res["Occupancy"] >= 3, (name, res)
