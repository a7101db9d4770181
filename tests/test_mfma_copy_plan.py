"""Host check of mfma_gemm's direct-to-LDS copy plan (CPU only).

tests/mfma_copy_check.cpp compiles tau.rs_amd/csrc/mfma_copy_plan.hpp, the
index helpers the kernel itself uses, with the host compiler and checks, for
the shipped 256x256 tile (4x4 waves of 64x64), the 128x128-wave-tile variant
(-DTAU_M256_BIG_WAVES, whose one GPU run faulted on a sign-extended address
word), the 128x128 and 64x256 tiles, both projections and both weight layouts,
at the c3, c5 prefill and c4 shapes plus an odd small one:
  * a scalar address split into two 32-bit words and joined again equals the
    original pointer, also when bit 31 of the low word is set;
  * one stage's copies write each LDS chunk of the A and B panels once and
    read each K chunk of each staged row once;
  * every per-lane offset at the last K step stays inside its tensor and fits
    the 32-bit offsets of the 128x128 wave tiles.
"""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_copy_plan_is_a_bijection_inside_the_tensors(tmp_path):
    exe = tmp_path / "mfma_copy_check"
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-o", str(exe),
                    os.path.join(ROOT, "tests", "mfma_copy_check.cpp")], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("ok ")
    assert int(r.stdout.split()[1]) > 1_000_000
