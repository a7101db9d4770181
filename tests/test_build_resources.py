"""Build-time resource checks of the prefill MFMA kernels (CPU only: hipcc
cross-compiles for gfx950).  A register spill inside the K loop turns every
step into scratch traffic with full waits, so the tiles are checked to
compile without spills, in the shipped configuration and in the optional
2x2-waves-of-128x128 one (-DTAU_M256_BIG_WAVES), whose 256 accumulators must
sit in AGPRs."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tau.rs_amd", "csrc", "grouped_gemm.hip")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def kernel_resources(tmp_path, defines):
    if not (os.path.exists(HIPCC) or shutil.which(HIPCC)):
        pytest.skip("hipcc not available")
    cmd = [HIPCC, "-std=c++17", "-O3", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-Wno-inline-asm", *defines, "--cuda-device-only", "-c", SRC,
           "-o", str(tmp_path / "gg.o"), "-Rpass-analysis=kernel-resource-usage"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    out, cur = {}, None
    for line in r.stderr.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur = m.group(1)
            out[cur] = {}
            continue
        m = re.search(r"remark:\s+(VGPRs|AGPRs|VGPRs Spill|SGPRs Spill|ScratchSize \[bytes/lane\]): (\d+)", line)
        if cur and m:
            out[cur][m.group(1)] = int(m.group(2))
    return out


BUILDS = {"default": [], "big_waves": ["-DTAU_M256_BIG_WAVES"], "split64": ["-DTAU_SPLIT_ROWS=64"],
          "frag_skip": ["-DTAU_FRAG_SKIP"]}


@pytest.fixture(scope="module")
def resources(tmp_path_factory):
    """Kernel resources of every build, compiled side by side."""
    import concurrent.futures
    dirs = {k: tmp_path_factory.mktemp(k) for k in BUILDS}
    with concurrent.futures.ThreadPoolExecutor(len(BUILDS)) as ex:
        futs = {k: ex.submit(kernel_resources, dirs[k], d) for k, d in BUILDS.items()}
        return {k: f.result() for k, f in futs.items()}


@pytest.mark.parametrize("build", list(BUILDS))
def test_mfma_tiles_compile_without_spills(resources, build):
    defines = BUILDS[build]
    res = resources[build]
    mfma = {k: v for k, v in res.items() if "mfma_gemm" in k}
    assert len(mfma) >= 20, sorted(res)
    for name, r in mfma.items():
        assert r.get("VGPRs Spill", 0) == 0 and r.get("SGPRs Spill", 0) == 0, (name, r)
        assert r.get("ScratchSize [bytes/lane]", 0) == 0, (name, r)
    big = {k: v for k, v in mfma.items() if "mfma_gemmILi256ELi256ELi2ELi2E" in k}
    if "-DTAU_M256_BIG_WAVES" in defines:
        assert big, "the 128x128 wave-tile kernels were not instantiated"
        for name, r in big.items():
            assert r["AGPRs"] >= 256, (name, r)  # accumulators in AGPRs
    else:
        assert not big
