"""The reference-compatible entry points (E=256, K=8), the elementwise and
linear entry points, the pointer-array and single-token decode entry points
and the separate shared-expert path, each called through the library's C ABI
on the CPU under the wavefront emulator (test infrastructure,
tests/wave_emu/abi_emu.cpp), with the cases of the GPU test
test_gpu_02_reference_abi.py (the reference tests each case follows are cited
there and per test below).  The oracle is the checker."""
import math
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "tests"))
GOLDEN = os.path.join(ROOT, "tests", "golden")

torch = pytest.importorskip("torch")

SOURCES = ["combine.cpp", "decode.cpp", "decode_layer.cpp", "decode_moe.cpp", "elementwise.cpp",
           "grouped_gemm.cpp", "moe.cpp", "norm.cpp", "router.cpp", "routing.cpp"]
E, K = 256, 8


@pytest.fixture(scope="module")
def exe(tmp_path_factory):
    import emu_build
    if not emu_build.available():
        pytest.skip("clang++ not available")
    work = tmp_path_factory.mktemp("abi_emu")
    return work, emu_build.build(work, "abi_emu.cpp", {"base": (SOURCES, [])})["base"]


def bf(a):
    """f32 values -> BF16 bit patterns (uint16)."""
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).view(torch.int16).numpy() \
        .view(np.uint16)


def unbf(b):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).float().numpy()


def rbf(a):
    """Round f32 values to BF16 and back."""
    return unbf(bf(a))


def call(exe, mode, ints, bufs):
    """Runs entry point `mode` with int arguments and buffers (numpy arrays, or
    None for a null pointer); returns (status, buffers after the call)."""
    work, binary = exe
    src, dst = work / "in.bin", work / "out.bin"
    with open(src, "wb") as f:
        f.write(np.array([mode, len(bufs), len(ints)], np.int32).tobytes())
        f.write(np.array(ints, np.int32).tobytes())
        for b in bufs:
            raw = b"" if b is None else np.ascontiguousarray(b).tobytes()
            f.write(np.int64(len(raw)).tobytes())
            f.write(raw)
    subprocess.run([str(binary), str(src), str(dst)], check=True, timeout=600)
    raw = np.fromfile(dst, np.uint8)
    status = int(raw[:4].view(np.int32)[0])
    out, o = [], 4
    for b in bufs:
        if b is None:
            out.append(None)
            continue
        n = b.nbytes
        out.append(raw[o:o + n].view(b.dtype).reshape(b.shape))
        o += n
    return status, out


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


# --- routing (components/cuda/routing.rs:80-160)

def test_routing_golden_rows_ties_and_nonfinite(exe, oracle):
    from safetensors.numpy import load_file
    d = load_file(os.path.join(GOLDEN, "moe_router_sm90.safetensors"))
    st, (_, routes) = call(exe, 0, [32], [bf(d["scores"]), np.zeros((32, 16), np.float32)])
    assert st == 0
    ids, w = d["ids"].astype(np.int64), d["weights"]
    np.testing.assert_array_equal(routes[:, :8].astype(np.int64), ids)
    assert np.all(np.abs(routes[:, 8:] - w) <= 1e-7 + 1e-5 * np.abs(w))
    oids, ow = oracle.route(rbf(d["scores"]), 8)
    np.testing.assert_array_equal(routes[:, 8:], ow)
    v = np.zeros((3, 256), np.float32)
    v[1, 7], v[2, 5] = np.nan, np.inf
    st, (_, routes) = call(exe, 0, [3], [bf(v), np.zeros((3, 16), np.float32)])
    assert st == 0 and routes[0, :8].tolist() == list(range(8)) and (routes[0, 8:] == np.float32(0.125)).all()
    assert np.isnan(routes[1:]).all()


# --- dispatch (components/cuda/fused_moe/prefill/tests.rs:43-120)

@pytest.mark.parametrize("tile_rows", [16, 32, 128])
def test_dispatch_long_to_short_reuse(exe, oracle, tile_rows):
    cap = oracle.capacity(257, E, K, tile_rows)
    ws = [np.zeros(514, np.int32), np.zeros(257, np.int32), np.zeros(cap, np.int32),
          np.zeros(cap // tile_rows, np.int32)]
    for tokens in [257, 1, 15, 16, 17, 31, 32, 33, 255, 256, 1]:
        for concentrated in (False, True):
            ids = np.array([[r if concentrated else (t * 8 + r) % 256 for r in range(8)] for t in range(tokens)])
            routes = np.concatenate([ids.astype(np.float32), np.full((tokens, 8), 0.125, np.float32)], 1)
            st, out = call(exe, 1, [tokens, cap, tile_rows], [routes] + ws)
            assert st == 0
            ws = out[1:]  # the next call reuses the workspace as left
            for got, ref in zip(ws, oracle.dispatch(ids, E, tile_rows, cap)):
                np.testing.assert_array_equal(got, ref)


def test_dispatch_invalid_routes_set_status(exe, oracle):
    cap = oracle.capacity(2, E, K, 16)
    routes = np.zeros((2, 16), np.float32)
    routes[0, :8] = np.arange(8)
    routes[1, :8] = [0, 1, 2, 3, 4, 5, 6, 6]  # duplicate expert in a token
    routes[:, 8:] = 0.125
    st, out = call(exe, 1, [2, cap, 16], [routes, np.zeros(514, np.int32), np.zeros(257, np.int32),
                                          np.zeros(cap, np.int32), np.zeros(cap // 16, np.int32)])
    assert st == 0 and out[1][512] == 1


# --- whole routed prefill (sparse_moe/tests/grouped.rs:7-200)

def reference_generator_layer(tokens, h, i):
    """The reference's deterministic grouped-prefill inputs (grouped.rs:40-114)."""
    values = lambda n, seed: (((np.arange(n) * 17 + seed) % 31).astype(np.float32) - 15.) / 128.
    router = np.zeros((E, h), np.float32)
    router[:, 0] = np.arange(E) / 32.
    data = values(tokens * h, 7).reshape(tokens, h)
    data[:, 0] = np.array([4., -4., 0.])[np.arange(tokens) % 3]
    return (data, data @ router.T, values(E * 2 * i * h, 1).reshape(E, 2 * i, h),
            values(E * h * i, 3).reshape(E, h, i))


@pytest.mark.parametrize("h,i", [(33, 17), (144, 80)])
def test_reference_prefill_parity(exe, oracle, h, i):
    for m in (16, 32):
        cap = oracle.capacity(257, E, K, m)
        for tokens in ((1, 257) if m == 16 else (17, 257)):
            x, logits, gu, dn = reference_generator_layer(tokens, h, i)
            bufs = [bf(x), bf(logits), bf(gu), bf(dn), np.zeros((257, 16), np.float32),
                    np.zeros(514, np.int32), np.zeros(257, np.int32), np.zeros(cap, np.int32),
                    np.zeros(cap // m, np.int32), np.zeros(1, np.uint16), np.zeros((cap, i), np.uint16),
                    np.zeros((257 * 8, h), np.uint16), np.zeros((tokens, h), np.uint16), np.zeros(10, np.int32)]
            st, out = call(exe, 2, [tokens, h, i, cap, m, 64 if m == 16 else 32, 64, 4, 2], bufs)
            assert st == 0
            ids, w = oracle.route(rbf(logits), K)
            np.testing.assert_array_equal(out[4][:tokens, :8].astype(np.int64), ids)
            xf, guf, dnf = rbf(x), rbf(gu), rbf(dn)
            ref16 = oracle.moe(xf, ids, w, guf, dnf, bf16=True)
            ref32 = oracle.moe(xf, ids, w, guf, dnf)
            got = unbf(out[12])
            assert rel_l2(got, ref16) <= 2e-3
            assert rel_l2(got, ref32) <= max(1e-2, rel_l2(ref16, ref32) + 1e-3)
            assert out[13][0] == m and out[13][5] == m  # the requested row block ran in both projections


@pytest.mark.parametrize("h,i", [(144, 80), (256, 64)])
def test_gate_up_projection_exact_on_dyadic_operands(exe, oracle, h, i):
    """moe_gemm.cu gate_up (down == 0) on the dyadic generator: exact at any
    summation order; padding rows are zero."""
    tokens = 33
    x, logits, gate_up, _ = reference_generator_layer(tokens, h, i)
    ids, _ = oracle.route(rbf(logits), K)
    for m in (16, 32, 64, 128, 256):
        meta, off, slots, tiles = oracle.dispatch(ids, E, m)
        cap = len(slots)
        routes = np.concatenate([ids.astype(np.float32), np.full((tokens, 8), 0.125, np.float32)], 1)
        bufs = [bf(x), bf(gate_up), routes, slots.astype(np.int32), tiles.astype(np.int32),
                np.full((cap, 2 * i), bf(np.float32(7.0)), np.uint16), np.zeros(5, np.int32)]
        st, out = call(exe, 3, [tokens, cap, 2 * i, h, 0, m, 64, 64, 4, 2], bufs)
        assert st == 0 and out[6][0] == m
        exp = np.zeros((cap, 2 * i), np.float32)
        xf, guf = rbf(x), rbf(gate_up)
        for row in range(cap):
            s_ = slots[row]
            if s_ < tokens * K:
                exp[row] = oracle.bf16_round(oracle.linear(xf[s_ // K][None], guf[ids.reshape(-1)[s_]])[0])
        np.testing.assert_array_equal(unbf(out[5]), exp)


def test_down_epilogue_weights_before_the_bf16_round(exe):
    """linear.rs:176-206: bf16(dot * w) with dot = 1 + 1/256, w = 0.9."""
    h, i = 2, 2
    routes = np.zeros((1, 16), np.float32)
    routes[0, :8] = np.arange(8)
    routes[0, 8] = 0.9
    a = np.zeros((128, i), np.float32)
    a[0] = [1.0, 1.0]
    down = np.zeros((E, h, i), np.float32)
    down[0, 0] = [1.0, 1.0 / 256.0]
    slots = np.full(128, 8, np.int32)
    tiles = np.full(8, -1, np.int32)
    for r in range(8):
        slots[16 * r], tiles[r] = r, r
    st, out = call(exe, 3, [1, 128, h, i, 1, 16, 16, 16, 1, 1],
                   [bf(a), bf(down), routes, slots, tiles, np.zeros((8, h), np.uint16), None])
    assert st == 0
    dot = np.float32(1 + 1 / 256)
    exact = rbf(np.float32(dot * np.float32(0.9)))
    early = rbf(rbf(dot) * rbf(np.float32(0.9)))
    assert exact != early and unbf(out[5])[0, 0] == exact


# --- elementwise and linear entry points

def test_silu_and_mul_vectors(exe):
    """silu_and_mul.rs:179-220: f32 within 1e-5, BF16 within 5e-2."""
    v = np.array([[1.0, -2.0, 0.5, 3.0, 2.0, 0.25, -4.0, 1.5],
                  [-0.5, 4.0, -3.0, 2.0, 1.25, -2.0, 0.75, 0.5]], np.float32)
    t = torch.tensor(v, dtype=torch.float64)
    ref = (torch.nn.functional.silu(t[:, :4]) * t[:, 4:]).numpy()
    st, out = call(exe, 4, [2, 4, 0], [v, np.zeros((2, 4), np.float32)])
    assert st == 0 and np.abs(out[1] - ref).max() <= 1e-5
    st, out = call(exe, 4, [2, 4, 1], [bf(v), np.zeros((2, 4), np.uint16)])
    assert st == 0 and np.abs(unbf(out[1]) - ref).max() <= 5e-2


@pytest.mark.parametrize("width", [2, 17, 2048])
def test_shared_combine_scalar_reference(exe, width):
    """shared_expert.rs:126-176: out == bf16(fma(gate, shared, routed)), gate
    from an f64 dot of the BF16 inputs."""
    inp = np.zeros(3 * width, np.float32)
    inp[0], inp[1], inp[2 * width] = 1., 1. / 256., -4.
    weight = np.zeros(width, np.float32)
    weight[0] = weight[1 % width] = 1.
    shared = np.array([((i % 13) - 6.) / 16. for i in range(3 * width)], np.float32)
    routed = np.array([((i % 17) - 8.) / 32. for i in range(3 * width)], np.float32)
    ins = [bf(a.reshape(3, width)) for a in (inp, shared, routed)]
    st, out = call(exe, 5, [3, width], [ins[0], bf(weight), ins[1], ins[2], np.zeros((3, width), np.uint16)])
    assert st == 0
    xi, s_, r_ = (unbf(a).astype(np.float64) for a in ins)
    wf = unbf(bf(weight)).astype(np.float64)
    for row in range(3):
        gate = np.float64(np.float32(1. / (1. + math.exp(-float((xi[row] * wf).sum())))))
        expected = rbf((gate * s_[row] + r_[row]).astype(np.float32))
        np.testing.assert_array_equal(unbf(out[4])[row], expected)


def test_linear_exact_on_dyadic_operands(exe):
    """linear.rs:117-172: the f32 projection equals the f64 dot bit for bit."""
    for rows, cols, inner in [(1, 1, 7), (3, 11, 16), (17, 19, 33), (5, 32, 64), (70, 130, 256)]:
        data = lambda n, seed: np.array([((i * 7 + seed) % 15 - 7) / 16. for i in range(n)], np.float32)
        x, w = data(rows * inner, 3).reshape(rows, inner), data(cols * inner, 5).reshape(cols, inner)
        st, out = call(exe, 6, [rows, cols, inner], [bf(x), bf(w), np.zeros((rows, cols), np.float32)])
        assert st == 0
        np.testing.assert_array_equal(out[2], (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32))


# --- decode entry points

def test_decode_gemm_pointer_arrays(exe):
    """moe_decode_gemm.cu pointer-array GEMV: out[b] = W[b] . x[b] in f32."""
    rng = np.random.default_rng(0)
    B, cols, inner = 8, 100, 96
    data = lambda *s: (rng.integers(-7, 8, size=s) / 16.).astype(np.float32)
    xs = [data(inner) for _ in range(B)]
    ws = [data(cols, inner) for _ in range(B)]
    st, out = call(exe, 7, [B, cols, inner, 2, 32, 128, 4, 2],
                   [bf(a) for a in xs] + [bf(a) for a in ws] + [np.zeros(cols, np.float32) for _ in range(B)])
    assert st == 0
    for b in range(B):
        np.testing.assert_array_equal(out[2 * B + b], (ws[b].astype(np.float64) @ xs[b]).astype(np.float32))


def test_fused_single_token_decode(exe, oracle):
    """fused_bf16_moe_decode.cu:56-91 contract vs the oracle (BF16 contract)."""
    rng = np.random.default_rng(1)
    h, i = 256, 64
    x, logits = rbf(rng.standard_normal(h)), rbf(rng.standard_normal(E))
    gu, dn = rbf(rng.standard_normal((E, 2 * i, h)) * 0.05), rbf(rng.standard_normal((E, h, i)) * 0.05)
    bufs = [bf(x), bf(logits), bf(gu), bf(dn), np.zeros(8, np.int32), np.zeros(8, np.float32),
            np.zeros(64, np.int64), np.zeros((8, 2 * i), np.uint16), np.zeros((8, i), np.uint16),
            np.zeros((8, h), np.uint16), np.zeros((8, 2 * i), np.float32), np.zeros((8, h), np.float32),
            np.zeros(h, np.uint16)]
    st, out = call(exe, 8, [h, i, E, K, 1, 64, 64, 4, 2], bufs)
    assert st == 0
    ids, w = oracle.route(logits[None], K)
    assert out[4].tolist() == ids[0].tolist()
    ref = oracle.moe(x[None], ids, w, gu, dn, bf16=True)[0]
    assert rel_l2(unbf(out[12]), ref) <= 2e-3


# --- the separate shared expert (shared_expert.rs:39-69,142-160; moe_shared.cu)

@pytest.mark.parametrize("tokens,layout", [(96, 1), (300, 0)])
def test_shared_expert_path(exe, oracle, tokens, layout):
    """routed + sigmoid(x . w_s) * mlp_s(x) at c4's sizes (hidden 2048, shared
    intermediate 512): against the oracle's BF16 contract and f32 path; 300
    tokens end in a partial row block of the dense shared GEMMs."""
    from frag16_host import frag16_permute
    H, Is = 2048, 512
    rng = np.random.default_rng(tokens)
    x = rbf(rng.standard_normal((tokens, H)))
    gu, dn = rbf(rng.standard_normal((2 * Is, H)) * 0.02), rbf(rng.standard_normal((H, Is)) * 0.02)
    gate_w, routed = rbf(rng.standard_normal(H) * 0.02), rbf(rng.standard_normal((tokens, H)) * 0.1)
    gub, dnb = bf(gu), bf(dn)
    if layout == 1:
        gub, dnb = frag16_permute(gub), frag16_permute(dnb)
    bufs = [bf(x), gub, dnb, bf(gate_w), bf(routed), np.zeros((tokens, Is), np.uint16),
            np.zeros((tokens, H), np.uint16), np.zeros((tokens, H), np.uint16), None]
    st, out = call(exe, 9, [tokens, H, Is, layout], bufs)
    assert st == 0
    got = unbf(out[7])
    ref16 = oracle.shared_combine_bf16(x, gate_w, oracle.dense_mlp(x, gu, dn, bf16=True), routed)
    ref32 = oracle.shared_combine_f32(x, gate_w, oracle.dense_mlp(x, gu, dn), routed)
    assert rel_l2(got, ref16) <= 2e-3
    assert rel_l2(got, ref32) <= 1e-2


@pytest.mark.parametrize("shape", [(3, 48, 128), (64, 192), (2, 1536, 2048)])
def test_pack_weights_matches_header_order(exe, shape):
    """tau_moe_pack_weights writes the FRAG16 order the header defines (its
    piece formula restated by frag16_host.frag16_permute, itself pinned to the
    literal loop in test_host)."""
    from frag16_host import frag16_permute
    rng = np.random.default_rng(len(shape))
    src = rng.integers(0, 1 << 16, size=shape, dtype=np.uint16)
    e, r, c = (1, *shape) if len(shape) == 2 else shape
    st, out = call(exe, 10, [e, r, c], [src, np.zeros_like(src)])
    assert st == 0
    np.testing.assert_array_equal(out[1], frag16_permute(src))
