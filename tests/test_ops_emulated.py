"""The router projection + routing and the fused residual add + centered
RMSNorm, run through the library's C ABI on the CPU under the wavefront
emulator (test infrastructure, tests/wave_emu/ops_emu.cpp), with the cases of
the GPU tests test_gpu_05_router_block.py and test_gpu_07_norm.py:
  * tau_launch_moe_router_route_ex on dyadic operands (every product and
    partial sum exact in f32, so the skinny MFMA projection's K order cannot
    matter): logits equal the oracle's x . W^T (+ bias) bit for bit, and the
    routes equal the oracle's routing of those logits bit for bit, for E up
    to 512 and K up to 32 (the reference's exact-dot test, components/cuda/
    linear.rs:117-172, and routing.rs:125-257);
  * tau_launch_fused_residual_rms_norm: the residual is the exact storage-dtype
    sum, the output is within one BF16 ulp (f32: 1e-6 + 2e-6|b|) of the f64
    closed form and of the f32 CPU oracle (the reference's rule,
    rms_norm/tests/residual/support.rs:22-42), equals the standalone norm of
    the residual bit for bit, and does not depend on the access-width policy."""
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "tests"))

torch = pytest.importorskip("torch")

SOURCES = ["combine.cpp", "decode.cpp", "decode_layer.cpp", "decode_moe.cpp", "elementwise.cpp",
           "grouped_gemm.cpp", "moe.cpp", "norm.cpp", "router.cpp", "routing.cpp"]


@pytest.fixture(scope="module")
def exe(tmp_path_factory):
    import emu_build
    if not emu_build.available():
        pytest.skip("clang++ not available")
    work = tmp_path_factory.mktemp("ops_emu")
    return work, emu_build.build(work, "ops_emu.cpp", {"base": (SOURCES, [])})["base"]


def bf16_bits(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).view(torch.int16).numpy() \
        .view(np.uint16)


def from_bits(b):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).float().numpy()


def invoke(exe, payload, tag):
    work, binary = exe
    src, dst = work / f"in_{tag}.bin", work / f"out_{tag}.bin"
    src.write_bytes(payload)
    subprocess.run([str(binary), str(src), str(dst)], check=True, timeout=600)
    raw = np.fromfile(dst, np.uint8)
    assert raw[:4].view(np.int32)[0] == 0, "launch status"
    return raw[4:]


def dyadic(shape, seed):
    n = int(np.prod(shape))
    return ((((np.arange(n) * 17 + seed) % 31).astype(np.float32) - 15.0) / 128.0).reshape(shape)


@pytest.mark.parametrize("t,h,e,k,bias", [(33, 160, 8, 2, False), (17, 96, 20, 4, True), (7, 256, 128, 8, True),
                                          (300, 256, 64, 6, True), (64, 2048, 128, 8, False),
                                          (40, 512, 512, 10, True), (5, 64, 256, 32, False)])
def test_router_route_exact_on_dyadic_operands(exe, oracle, t, h, e, k, bias):
    x, w = dyadic((t, h), 3), dyadic((e, h), 5)
    b = (np.arange(e, dtype=np.float32) - e / 2) / 64.0 if bias else np.zeros(e, np.float32)
    hdr = np.array([0, t, h, e, k, int(bias)], np.int32)
    out = invoke(exe, hdr.tobytes() + bf16_bits(x).tobytes() + bf16_bits(w).tobytes() + b.tobytes(), "router")
    logits = out[:t * e * 4].view(np.float32).reshape(t, e)
    routes = out[t * e * 4:].view(np.float32).reshape(t, 2 * k)
    ref = oracle.linear(x, w) + (b[None, :] if bias else 0)
    np.testing.assert_array_equal(logits, ref)
    ids, wts = oracle.route(ref, k)
    np.testing.assert_array_equal(routes[:, :k].astype(np.int64), ids)
    np.testing.assert_array_equal(routes[:, k:], wts)


def run_norm(exe, oracle, rows, cols, bf16, policy=16, eps=1e-6):
    from norm_host import assert_close, f64_norm, patterned, to_dtype
    n = rows * cols
    x, b, w = (to_dtype(patterned(n, 3), bf16).reshape(rows, cols), to_dtype(patterned(n, 19), bf16).reshape(rows, cols),
               to_dtype(patterned(cols, 47), bf16))
    enc = bf16_bits if bf16 else (lambda a: np.ascontiguousarray(a, np.float32))
    hdr = np.array([1, rows, cols, int(bf16), policy], np.int32).tobytes() + np.float32(eps).tobytes()
    out = invoke(exe, hdr + enc(x).tobytes() + enc(b).tobytes() + enc(w).tobytes(), "norm")
    es = 2 if bf16 else 4
    parts = [out[i * n * es:(i + 1) * n * es] for i in range(3)]
    dec = (lambda p: from_bits(p.view(np.uint16))) if bf16 else (lambda p: p.view(np.float32).copy())
    res, y, alone = (dec(p).reshape(rows, cols) for p in parts)
    ref_res, ref_y = oracle.centered_rms_norm(x, w, eps, branch=b, bf16=bf16)
    np.testing.assert_array_equal(res, ref_res)
    assert_close(y, f64_norm(ref_res, w, eps), bf16)
    if cols <= 5120:
        assert_close(y, ref_y, bf16)
    np.testing.assert_array_equal(parts[1], parts[2])  # fused output == norm(residual), bit for bit
    return parts[1]


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
def test_norm_widths_and_wide_rows(exe, oracle, bf16):
    for cols in [1, 31, 32, 33, 255, 256, 257, 2560, 5120]:
        for rows in [1, 5]:
            run_norm(exe, oracle, rows, cols, bf16)
    for cols in [9000, 20000]:  # more than 16 chunks of 16 bytes per lane: the recompute path
        run_norm(exe, oracle, 3, cols, bf16)


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
def test_norm_policies_give_identical_bits(exe, oracle, bf16):
    for cols in [256, 2560, 5120]:
        outs = [run_norm(exe, oracle, 2, cols, bf16, policy=p) for p in (0, 4, 8, 16)]
        for o in outs[1:]:
            np.testing.assert_array_equal(o, outs[0])
