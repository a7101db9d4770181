"""The library's routing kernels, run on the CPU under a wavefront emulator,
against the oracle (CPU; no GPU needed).

tests/wave_emu/route_emu.cpp compiles the routing launchers (routing.hip:
route_kernel, route_shared_kernel from dispatch.hpp) with the host compiler
and executes each 64-lane wavefront with one thread per lane and the
cross-lane operations (DPP moves, shuffles) of tests/wave_emu/hip/hip_runtime.h.  This
checks the routing algorithm itself (the f32 softmax with glibc's exp bits,
the denominator summed in expert order, ranking on probabilities with the
lower id on ties, the rank-ordered renormalisation, the unnormalised and
shared-expert variants, rejected rows) bit for bit against the oracle's
restatement of routing.rs:125-257, on the same cases as the GPU tests.  The
GPU tests (test_gpu_01_parity.py) run the same kernels on the hardware."""
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def emu(tmp_path_factory):
    import emu_build
    if not emu_build.available():
        pytest.skip("clang++ not available")
    work = tmp_path_factory.mktemp("emu")
    exe = emu_build.build(work, "route_emu.cpp", {"route": (["routing.cpp"], [])})["route"]

    def run(logits, k, bf16=False, normalize=True, shared=False):
        lg = np.ascontiguousarray(logits, np.float32)
        t, width = lg.shape
        e = width - (1 if shared else 0)
        dtype = (1 if bf16 else 0) | (0 if normalize else 0x100)
        hdr = np.array([t, e, k, dtype, int(shared)], np.int32)
        if bf16:
            bits = lg.view(np.uint32)
            assert np.all(bits & 0xFFFF == 0), "BF16 logits must be BF16-representable"
            payload = (bits >> 16).astype(np.uint16).tobytes()
        else:
            payload = lg.tobytes()
        src, dst = work / "in.bin", work / "out.bin"
        src.write_bytes(hdr.tobytes() + payload)
        subprocess.run([str(exe), str(src), str(dst)], check=True, timeout=300)
        raw = np.fromfile(dst, np.float32)
        assert raw[:1].view(np.int32)[0] == 0, "launch status"
        return raw[1:].reshape(t, -1)

    return run


def bf16_round(a):
    from oracle import oracle
    return oracle.bf16_round(np.asarray(a, np.float32))


def test_golden_router_rows(emu, oracle):
    from safetensors.numpy import load_file
    d = load_file(os.path.join(ROOT, "tests", "golden", "moe_router_sm90.safetensors"))
    scores, ids_ref = d["scores"], d["ids"].astype(np.int64)
    r = emu(scores, 8)
    np.testing.assert_array_equal(r[:, :8].astype(np.int64), ids_ref)
    ids, w = oracle.route(scores, 8)
    np.testing.assert_array_equal(r[:, 8:], w)
    assert np.all(np.abs(r[:, 8:] - d["weights"]) <= 1e-7 + 1e-5 * np.abs(d["weights"]))


@pytest.mark.parametrize("E,K", [(8, 2), (128, 8), (512, 10)])
def test_near_max_ulp_ties(emu, oracle, E, K):
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    rng = np.random.default_rng(E + K)
    near = np.array([0.0, -2.0 ** -25, -2.0 ** -24, -2.0 ** -23], np.float32)
    rows = []
    for _ in range(8):
        base = np.minimum(rng.standard_normal(E) * 2 - 8, -1).astype(np.float32)
        base[rng.choice(E, 4, replace=False)] = rng.permutation(near)
        rows.append(base)
    lg = np.stack(rows)
    r = emu(lg, K)
    ids, w = oracle.route(lg, K)
    np.testing.assert_array_equal(r[:, :K].astype(np.int64), ids)
    np.testing.assert_array_equal(r[:, K:], w)
    # the lower id wins against a larger logit somewhere (the case the old logit key got wrong)
    assert any(lg[t, ids[t, i]] < lg[t, ids[t, i + 1]] for t in range(len(lg)) for i in range(K - 1))


@pytest.mark.parametrize("E,K,bf16", [(64, 32, True), (512, 20, True), (512, 32, False), (200, 16, True),
                                      (200, 12, False), (48, 17, False), (256, 8, True)])
def test_coarse_ties_wide_top_k(emu, oracle, E, K, bf16):
    rng = np.random.default_rng(100 + E + K)
    lg = (rng.integers(-6, 7, (9, E)) * 0.25).astype(np.float32)
    r = emu(lg, K, bf16=bf16)
    ids, w = oracle.route(lg, K)
    np.testing.assert_array_equal(r[:, :K].astype(np.int64), ids)
    np.testing.assert_array_equal(r[:, K:], w)


@pytest.mark.parametrize("bf16", [False, True])
def test_unnormalised_weights_and_benchmark_shapes(emu, oracle, bf16):
    rng = np.random.default_rng(7)
    for E, K in [(128, 8), (8, 2), (512, 10)]:
        lg = (rng.standard_normal((12, E)) * 1.5).astype(np.float32)
        if bf16:
            lg = bf16_round(lg)
        for normalize in (True, False):
            r = emu(lg, K, bf16=bf16, normalize=normalize)
            ids, w = oracle.route(lg, K, normalize=normalize)
            np.testing.assert_array_equal(r[:, :K].astype(np.int64), ids)
            np.testing.assert_array_equal(r[:, K:], w)


def test_shared_expert_rank(emu, oracle):
    rng = np.random.default_rng(3)
    E, K = 96, 6
    lg = (rng.standard_normal((10, E + 1)) * 2).astype(np.float32)
    r = emu(lg, K, shared=True)
    ids, w = oracle.route(lg[:, :E], K)
    K1 = K + 1
    np.testing.assert_array_equal(r[:, :K].astype(np.int64), ids)
    np.testing.assert_array_equal(r[:, K1:K1 + K], w)
    assert np.all(r[:, K] == E)
    np.testing.assert_array_equal(r[:, K1 + K], oracle.sigmoid(lg[:, E]))


def test_rejected_rows_and_closed_forms(emu):
    lg = np.zeros((6, 256), np.float32)
    lg[2, 17] = np.nan
    lg[4, 0] = np.inf
    r = emu(lg, 8)
    for t in (2, 4):
        assert np.all(np.isnan(r[t]))
    for t in (0, 1, 3, 5):  # uniform rows: ids 0..7, weights 1/8
        assert list(r[t, :8]) == list(range(8)) and np.all(r[t, 8:] == np.float32(0.125))
