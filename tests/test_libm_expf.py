"""The routing exp (csrc/libm_expf.hpp) equals glibc's expf on every float.

The reference's f32 CPU routing ranks experts by f32 softmax probabilities
computed with Rust's f32::exp (glibc expf on linux-gnu;
crates/models/src/components/sparse_moe/routing.rs:139-141,239-257), so the
GPU routing kernels use an exp with the same bits.  The header is compiled for
the host here and compared with the C library's expf over all 2^32 bit
patterns (NaNs skipped)."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_expf_glibc_matches_system_expf_on_every_float(tmp_path):
    exe = tmp_path / "libm_expf_check"
    subprocess.run(["g++", "-std=c++17", "-O2", "-fopenmp", "-o", str(exe),
                    os.path.join(ROOT, "tests", "libm_expf_check.cpp"), "-lm"], check=True)
    r = subprocess.run([str(exe), "1"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0" in r.stdout
    checked = int(r.stdout.split()[1])
    assert checked == (1 << 32) - 2 * ((1 << 23) - 1)  # every non-NaN pattern
