"""The fused decode path, run on the CPU under the wavefront emulator
(test infrastructure, tests/wave_emu), against the oracle and across builds.

tests/wave_emu/decode_emu.cpp calls the library's own launch_decode_moe
(routing, the two weight-streaming projection kernels with the plan workgroup,
the combine; decode_moe.hip) on small layers, and the same with
-DTAU_DECODE_ONE_LAUNCH (the one-launch layer of decode_layer.hip, off in the
shipped build).  Checks:
  * routes equal the oracle's bit for bit; the dispatch plan equals the
    oracle's stable dispatch; the output is within the BF16 contract's
    tolerance of the oracle (the emulator sums each MFMA's K in order, the
    hardware in its own order, so no bit-level claim is made there);
  * the one-launch layer reproduces every buffer of the two-launch path bit
    for bit (routes, plan, activated, contributions, output): the two issue
    the same MFMA sequence per output element, so any difference is a bug in
    the new kernel's row lists, LDS staging, splits or plan.
The GPU tests run both on the hardware (test_gpu_03_decode_path.py)."""
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "tests"))

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def bins(tmp_path_factory):
    import emu_build
    if not emu_build.available():
        pytest.skip("clang++ not available")
    work = tmp_path_factory.mktemp("decode_emu")
    srcs = ["routing.cpp", "combine.cpp", "decode_moe.cpp", "decode_layer.cpp"]
    return work, emu_build.build(work, "decode_emu.cpp", {"two": (srcs, []),
                                                         "one": (srcs, ["-DTAU_DECODE_ONE_LAUNCH"])})


def bf16_bits(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).view(torch.int16).numpy() \
        .view(np.uint16)


def from_bits(b):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).float().numpy()


def run(bins, which, x, logits, gu, dn, layout, bf16_logits=True, raw=False):
    work, exe = bins
    T, H = x.shape
    E, two_i, _ = gu.shape
    I = two_i // 2
    K = run.K
    ldt = (1 if bf16_logits else 0) | (0x100 if raw else 0)
    key = (id(x), id(logits), id(gu), id(dn), layout, ldt, K)
    src, dst = work / "in.bin", work / f"out_{which}.bin"
    if run.encoded != key:  # both builds read the same encoded input
        from frag16_host import frag16_permute
        gu_b, dn_b = bf16_bits(gu), bf16_bits(dn)
        if layout == 1:
            gu_b, dn_b = frag16_permute(gu_b), frag16_permute(dn_b)
        lg = bf16_bits(logits) if bf16_logits else np.ascontiguousarray(logits, np.float32)
        hdr = np.array([T, H, I, E, K, layout, ldt], np.int32)
        with open(src, "wb") as f:
            for part in (hdr, bf16_bits(x), lg, gu_b, dn_b):
                f.write(memoryview(np.ascontiguousarray(part)).cast("B"))
        run.encoded = key
    if which is None:
        return None
    subprocess.run([str(exe[which]), str(src), str(dst)], check=True, timeout=900)
    raw_out = np.fromfile(dst, np.uint8)
    o = 0

    def take(dtype, n):
        nonlocal o
        v = raw_out[o:o + n * np.dtype(dtype).itemsize].view(dtype)
        o += n * np.dtype(dtype).itemsize
        return v

    status, cap = take(np.int32, 2)
    assert status == 0
    return {"routes": take(np.float32, T * 2 * K).reshape(T, 2 * K), "meta": take(np.int32, 2 * E + 2),
            "offsets": take(np.int32, E + 1), "slots": take(np.int32, cap), "tiles": take(np.int32, cap // 16),
            "activated": take(np.uint16, T * K * I), "contributions": take(np.uint16, T * K * H),
            "output": take(np.uint16, T * H).reshape(T, H), "cap": int(cap)}


def banks(rng, shape):
    """BF16-exact expert weights ~N(0, 0.05^2).  Full-size banks (about a
    gigabyte) take each expert's matrix as a different shifted window of one
    random pool, so every expert still holds different values at every
    position while generation stays a few seconds."""
    E, n = shape[0], shape[1] * shape[2]
    if E * n <= 1 << 24:
        return from_bits(bf16_bits(rng.standard_normal(shape) * 0.05))
    step = 4099
    pool = from_bits(bf16_bits(rng.standard_normal(n + E * step).astype(np.float32) * 0.05))
    out = np.empty((E, n), np.float32)
    for e in range(E):
        out[e] = pool[e * step:e * step + n]
    return out.reshape(shape)


CASES = [  # T, H, I, E, K, layout, bf16 logits, raw weights, NaN row, tied logits
    (16, 256, 256, 8, 2, 1, True, False, False, False),
    (5, 256, 512, 16, 4, 0, False, False, False, False),
    (12, 256, 256, 24, 3, 1, True, True, False, False),
    (8, 256, 256, 8, 2, 1, True, False, True, False),
    (64, 256, 256, 32, 8, 1, True, False, False, False),  # skewed below: experts with 17-64 rows (row groups 2-4)
    (64, 2048, 768, 128, 8, 1, True, False, False, False),  # the c2 (Qwen3-30B-A3B decode) layer at full size
    (16, 256, 512, 8, 2, 1, False, False, False, False),  # the c1 tiny layer's shape, f32 router logits
    (32, 4096, 1536, 16, 8, 1, True, False, False, False),  # c5 decode's sizes (H 4096, I 1536, 32 tokens), 16 experts
    (24, 256, 128, 60, 20, 0, True, False, False, True),  # E not a multiple of 8, K > 16, heavy ties
    (40, 256, 128, 128, 8, 1, False, False, False, True),  # f32 logits on a coarse grid
    (64, 256, 64, 250, 3, 1, True, False, False, False),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_decode_path_emulated(bins, oracle, case):
    T, H, I, E, K, layout, bf16_logits, raw, nan_row, ties = CASES[case]
    rng = np.random.default_rng(40 + case)
    x = from_bits(bf16_bits(rng.standard_normal((T, H))))
    gu = banks(rng, (E, 2 * I, H))
    dn = banks(rng, (E, H, I))
    logits = (rng.standard_normal((T, E)) * 2).astype(np.float32)
    if ties:  # a coarse grid: many equal logits per row, broken by expert id
        logits = np.round(logits * 4) / 4
    if bf16_logits:
        logits = from_bits(bf16_bits(logits))
    if nan_row:
        logits[3, 1] = np.nan
    if T == 64 and E == 32:  # a per-expert popularity bias: some experts take most tokens
        logits = logits + (rng.standard_normal(E) * 1.5).astype(np.float32)
        if bf16_logits:
            logits = from_bits(bf16_bits(logits))
    run.K = K
    run.encoded = None
    run(bins, None, x, logits, gu, dn, layout, bf16_logits, raw)  # encode the input once
    import concurrent.futures
    # The one-launch layer recomputes gate_up per split (4 splits below 64
    # experts): at the large sizes with few experts only the shipped path runs.
    builds = ("two",) if H >= 2048 and E < 64 else ("two", "one")
    with concurrent.futures.ThreadPoolExecutor(2) as ex:
        res = list(ex.map(lambda v: run(bins, v, x, logits, gu, dn, layout, bf16_logits, raw), builds))
    two, one = res[0], res[-1]
    for key in ("routes", "meta", "offsets", "slots", "tiles", "contributions", "output"):
        np.testing.assert_array_equal(one[key].view(np.uint32) if one[key].dtype == np.float32 else one[key],
                                      two[key].view(np.uint32) if two[key].dtype == np.float32 else two[key],
                                      err_msg=key)
    # activated: the assignment rows the layer wrote (every assignment of a valid row)
    valid_rows = ~np.isnan(two["routes"][:, 0])
    a_rows = np.flatnonzero(np.repeat(valid_rows, K))
    np.testing.assert_array_equal(one["activated"].reshape(T * K, I)[a_rows],
                                  two["activated"].reshape(T * K, I)[a_rows])
    if nan_row:
        assert two["meta"][2 * E] == 1 and np.all(np.isnan(from_bits(two["output"])))
        return
    if T == 64 and E == 32:
        assert two["meta"][:E].max() > 32  # several 16-row groups for one expert
    ids, w = oracle.route(logits, K, normalize=not raw)
    np.testing.assert_array_equal(two["routes"][:, :K].astype(np.int64), ids)
    np.testing.assert_array_equal(two["routes"][:, K:], w)
    meta, offsets, slots, tiles = oracle.dispatch(ids, E, 16, two["cap"])
    np.testing.assert_array_equal(two["meta"], meta)
    np.testing.assert_array_equal(two["offsets"], offsets)
    np.testing.assert_array_equal(two["slots"], slots)
    np.testing.assert_array_equal(two["tiles"], tiles)
    ref = oracle.moe(x, ids, w, gu, dn, bf16=True)
    got = from_bits(two["output"])
    err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert err <= 2e-3, err
