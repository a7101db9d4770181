"""The whole routed layer through the C ABI (tau_launch_moe_prefill_ex),
run on the CPU under the wavefront emulator (test infrastructure,
tests/wave_emu), for the shipped build and the off-by-default tile variants.

tests/wave_emu/prefill_emu.cpp links every library source, rewritten by
tests/wave_emu/prep.py (the direct-to-LDS copy's inline assembly becomes the
emulator's copy with the same per-lane source and LDS destination; the
32x32x16 and 16x16x32 MFMAs are computed in f32), and runs routing, dispatch,
the grouped MFMA projections and the combine on small layers whose skewed
routing gives both full and nearly empty 256-row blocks.  Checks:
  * the shipped build: routes and the dispatch plan equal the oracle's bit
    for bit, the output is within the BF16 contract's tolerance of the oracle
    (the emulator's MFMA sums K in order; the hardware's order is not claimed);
  * -DTAU_M256_BIG_WAVES (2x2 waves of 128x128: 32-bit copy offsets from a
    scalar base, the variant whose one GPU run faulted),
    -DTAU_SPLIT_ROWS=32 / 64 / 128 (lightly filled blocks on the
    weight-streaming kernel or the shorter MFMA tile in a second launch) and
    the 128x128 tiles with the 64-row split, and -DTAU_FRAG_SKIP (the shipped
    tile skipping padding per 32-row fragment) reproduce the shipped build's activated rows, contributions
    and output bit for bit: per output element they issue the same MFMA
    sequence, so any difference is an addressing or scheduling bug (the
    32-row split computes its blocks with 16x16x32 MFMAs, whose internal
    summation order on the hardware may differ from 32x32x16's; under the
    emulator both sum K in order, so the comparison still isolates its
    addressing)."""
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
VARIANTS = {"base": [], "bigwaves": ["-DTAU_M256_BIG_WAVES"], "split64": ["-DTAU_SPLIT_ROWS=64"],
            "split128": ["-DTAU_SPLIT_ROWS=128"], "split32": ["-DTAU_SPLIT_ROWS=32"],
            "bigwaves_split64": ["-DTAU_M256_BIG_WAVES", "-DTAU_SPLIT_ROWS=64"], "fragskip": ["-DTAU_FRAG_SKIP"],
            "bigwaves_noskip": ["-DTAU_M256_BIG_WAVES", "-DTAU_BIG_WAVE_NO_SKIP"]}


@pytest.fixture(scope="module")
def bins(tmp_path_factory):
    import emu_build
    if not emu_build.available():
        pytest.skip("clang++ not available")
    work = tmp_path_factory.mktemp("prefill_emu")
    return work, emu_build.build(work, "prefill_emu.cpp", {k: (SOURCES, v) for k, v in VARIANTS.items()})


def bf16_bits(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).view(torch.int16).numpy() \
        .view(np.uint16)


def from_bits(b):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).float().numpy()


def run(bins, which, x, logits, gu, dn, K, M, layout, bf16_logits=True, shared=0):
    """shared=1: gu/dn hold the shared expert as expert E and logits its gate
    column last; the routes then have K+1 picks."""
    work, exe = bins
    T, H = x.shape
    E, two_i, _ = gu.shape
    E -= shared
    I = two_i // 2
    from frag16_host import frag16_permute
    gu_b, dn_b = bf16_bits(gu), bf16_bits(dn)
    if layout == 1:
        gu_b, dn_b = frag16_permute(gu_b), frag16_permute(dn_b)
    lg = bf16_bits(logits) if bf16_logits else np.ascontiguousarray(logits, np.float32)
    hdr = np.array([T, H, I, E, K, M, layout, 1 if bf16_logits else 0, shared], np.int32)
    src, dst = work / f"in_{which}.bin", work / f"out_{which}.bin"
    src.write_bytes(hdr.tobytes() + bf16_bits(x).tobytes() + lg.tobytes() + gu_b.tobytes() + dn_b.tobytes())
    subprocess.run([str(exe[which]), str(src), str(dst)], check=True, timeout=900)
    raw = np.fromfile(dst, np.uint8)
    o = 0

    def take(dtype, n):
        nonlocal o
        v = raw[o:o + n * np.dtype(dtype).itemsize].view(dtype)
        o += n * np.dtype(dtype).itemsize
        return v

    status, cap = take(np.int32, 2)
    assert status == 0, status
    E, K = E + shared, K + shared
    return {"routes": take(np.float32, T * 2 * K).reshape(T, 2 * K), "meta": take(np.int32, 2 * E + 2),
            "offsets": take(np.int32, E + 1), "slots": take(np.int32, cap), "tiles": take(np.int32, cap // M),
            "activated": take(np.uint16, cap * I).reshape(cap, I), "contributions": take(np.uint16, T * K * H),
            "output": take(np.uint16, T * H).reshape(T, H), "cap": int(cap),
            "counts": dict(zip(("mfma16", "mfma32", "dma16"), take(np.int64, 3).tolist()))}


def layer(seed, T, H, I, E, skew=True):
    rng = np.random.default_rng(seed)
    x = from_bits(bf16_bits(rng.standard_normal((T, H))))
    gu = from_bits(bf16_bits(rng.standard_normal((E, 2 * I, H)) * 0.05))
    dn = from_bits(bf16_bits(rng.standard_normal((E, H, I)) * 0.05))
    logits = rng.standard_normal((T, E)).astype(np.float32)
    if skew:  # expert 0 takes most tokens: full 256-row blocks beside nearly empty ones
        logits[:, 0] += 3.0
    return x, logits, gu, dn


def check_against_oracle(oracle, res, x, logits, gu, dn, K, M, bf16_logits=True):
    E = gu.shape[0]
    lg = from_bits(bf16_bits(logits)) if bf16_logits else logits
    ids, w = oracle.route(lg, K)
    np.testing.assert_array_equal(res["routes"][:, :K].astype(np.int64), ids)
    np.testing.assert_array_equal(res["routes"][:, K:], w)
    meta, offsets, slots, tiles = oracle.dispatch(ids, E, M, res["cap"])
    np.testing.assert_array_equal(res["meta"], meta)
    np.testing.assert_array_equal(res["offsets"], offsets)
    np.testing.assert_array_equal(res["slots"], slots)
    np.testing.assert_array_equal(res["tiles"], tiles)
    ref = oracle.moe(x, ids, w, gu, dn, bf16=True)
    got = from_bits(res["output"])
    err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert err <= 2e-3, err
    return meta


@pytest.mark.parametrize("layout", [1, 0])
def test_256_row_tiles_and_variants(bins, oracle, layout):
    T, H, I, E, K = 160, 256, 256, 8, 2
    x, logits, gu, dn = layer(11 + layout, T, H, I, E)
    base = run(bins, "base", x, logits, gu, dn, K, 256, layout)
    meta = check_against_oracle(oracle, base, x, logits, gu, dn, K, 256)
    counts = meta[:E]
    assert counts.max() > 128 and (counts[counts > 0] <= 64).any()  # both kinds of block
    for v in ("bigwaves", "split32", "split64", "split128", "bigwaves_split64", "fragskip"):
        res = run(bins, v, x, logits, gu, dn, K, 256, layout)
        for key in ("routes", "meta", "slots", "tiles", "contributions", "output"):
            np.testing.assert_array_equal(res[key].view(np.uint32) if res[key].dtype == np.float32 else res[key],
                                          base[key].view(np.uint32) if base[key].dtype == np.float32 else base[key],
                                          err_msg=f"{v}: {key}")
        live = base["slots"] < T * K  # rows holding an assignment (padding and dead rows are layout details)
        np.testing.assert_array_equal(res["activated"][live], base["activated"][live], err_msg=f"{v}: activated")


@pytest.mark.parametrize("M,layout,bf16_logits", [(16, 1, True), (32, 0, True), (64, 0, False), (128, 1, True)])
def test_shorter_tiles(bins, oracle, M, layout, bf16_logits):
    """16/32-row blocks: the weight-streaming grouped kernels (96 tokens, so not
    the fused decode path); 64/128: the shorter MFMA tiles."""
    T, H, I, E, K = 96, 256, 192, 6, 3
    x, logits, gu, dn = layer(20 + M, T, H, I, E)
    if layout == 1:  # FRAG16 needs I % 64 == 0
        x, logits, gu, dn = layer(20 + M, T, H, 256, E)
    res = run(bins, "base", x, logits, gu, dn, K, M, layout, bf16_logits)
    check_against_oracle(oracle, res, x, logits, gu, dn, K, M, bf16_logits)


@pytest.mark.parametrize("H,I,T", [(2048, 768, 346), (4096, 1536, 272)], ids=["c3_dims", "c5p_dims"])
def test_benchmark_layer_dims(bins, oracle, H, I, T):
    """The 256-row MFMA tile at the hidden and intermediate sizes of the
    30B-A3B (c3) and 235B-A22B (c5 prefill) layers: full-length K loops
    (32 / 64 steps of 64), the real operand strides, and a skewed expert with
    one full and one nearly empty block.  Three experts keep the emulated work
    to a few GFLOP.  The shipped build is checked against the oracle, the
    128x128 wave-tile build bit for bit against it."""
    import concurrent.futures
    E, K = 3, 2
    x, logits, gu, dn = layer(5, T, H, I, E)
    with concurrent.futures.ThreadPoolExecutor(3) as ex:
        futs = {v: ex.submit(run, bins, v, x, logits, gu, dn, K, 256, 1) for v in ("base", "bigwaves", "fragskip")}
        res = {v: f.result() for v, f in futs.items()}
    meta = check_against_oracle(oracle, res["base"], x, logits, gu, dn, K, 256)
    assert meta[0] > 256 and meta[0] % 256 <= 96  # a full block and a partly empty one
    # 128-row wave tiles see 0 to 4 live 32-row fragments across the blocks
    # (c3 sizes: about 90 rows in expert 0's second block -> 3, about 173 rows in the others -> 4 and 2)
    for v in ("bigwaves", "fragskip"):
        for key in ("routes", "slots", "contributions", "output"):
            np.testing.assert_array_equal(res[v][key], res["base"][key], err_msg=f"{v}: {key}")


def test_folded_shared_expert_c4_dims(bins, oracle):
    """The c4 layer's always-on shared expert folded into the routed schedule
    (tau_launch_moe_routing_shared_ex, then tau_launch_moe_prefill_ex from the
    routes with E+1 experts and K+1 picks) at c4's hidden and intermediate
    sizes (2048, 512), 16 routed experts, top-4, 256 tokens on 256-row tiles
    (the shared expert fills a whole block).  Routed ranks equal the oracle's
    routing bit for bit and rank K is (E, sigmoid(gate)); the output is within
    the BF16 contract's tolerance of the oracle run as E+1 experts, and within
    the north-star tolerance of the reference's f32 path with the separate
    shared combine (routed + sigmoid(x . w_s) * mlp_s(x), shared_expert.rs:39-69)."""
    T, H, I, E, K = 256, 2048, 512, 16, 4
    x, logits, gu, dn = layer(31, T, H, I, E + 1)
    rng = np.random.default_rng(32)
    w_s = rng.standard_normal(H).astype(np.float32) * 0.02
    logits[:, E] = x @ w_s  # the shared gate logit x . w_s, last column
    res = run(bins, "base", x, logits, gu, dn, K, 256, 1, bf16_logits=False, shared=1)
    ids, w = oracle.route(logits[:, :E], K)
    gate = oracle.sigmoid(logits[:, E])
    r = res["routes"]
    np.testing.assert_array_equal(r[:, :K].astype(np.int64), ids)
    np.testing.assert_array_equal(r[:, K + 1:2 * K + 1], w)
    assert np.all(r[:, K] == E)
    np.testing.assert_array_equal(r[:, 2 * K + 1], gate)
    ids_x = np.concatenate([ids, np.full((T, 1), E, np.int64)], 1)
    w_x = np.concatenate([w, gate[:, None]], 1).astype(np.float32)
    meta, offsets, slots, tiles = oracle.dispatch(ids_x, E + 1, 256, res["cap"])
    np.testing.assert_array_equal(res["meta"], meta)
    np.testing.assert_array_equal(res["slots"], slots)
    got = from_bits(res["output"])
    ref_bf16 = oracle.moe(x, ids_x, w_x, gu, dn, bf16=True)
    assert np.linalg.norm(got - ref_bf16) / np.linalg.norm(ref_bf16) <= 2e-3
    routed = oracle.moe(x, ids, w, gu[:E], dn[:E])
    ref = oracle.shared_combine_f32(x, w_s, oracle.dense_mlp(x, gu[E], dn[E]), routed)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-2


@pytest.mark.parametrize("T,E,K,shared,bias", [(4096, 128, 8, 0, "normal"), (2048, 512, 10, 1, "zipf"),
                                               (8192, 128, 8, 0, "none")], ids=["c3", "c4", "c5p"])
def test_full_size_routing_and_dispatch(bins, oracle, tau, T, E, K, shared, bias):
    """Routing and the multi-workgroup dispatch (32 chunks of whole 64-token
    passes) at the benchmark layers' token, expert and top-k counts, with the
    row block the library selects for the real hidden/intermediate sizes:
    c3's per-expert N(0,1) router bias, c4's Zipf(1.1) popularity bias with the
    shared expert folded in as expert 512, c5 prefill's uniform routing.
    Hidden and intermediate are 64 so the projections stay cheap; routes,
    meta, offsets, slots and tiles must equal the oracle's bit for bit (the
    reference's stable token-ascending order, routing.rs:159-227), and the
    output is checked against the oracle's BF16 contract."""
    dims = {"c3": (2048, 768), "c4": (2048, 512), "c5p": (4096, 1536)}
    H, I = 64, 64
    rng = np.random.default_rng(T + E)
    x = from_bits(bf16_bits(rng.standard_normal((T, H))))
    gu = from_bits(bf16_bits(rng.standard_normal((E + shared, 2 * I, H)) * 0.05))
    dn = from_bits(bf16_bits(rng.standard_normal((E + shared, H, I)) * 0.05))
    logits = rng.standard_normal((T, E + shared)).astype(np.float32)
    if bias == "normal":
        logits[:, :E] += rng.standard_normal(E).astype(np.float32)
    elif bias == "zipf":
        logits[:, :E] += np.log(1.0 / np.arange(1, E + 1) ** 1.1)[rng.permutation(E)].astype(np.float32)
    logits = from_bits(bf16_bits(logits))
    real_h, real_i = dims["c3" if T == 4096 else "c4" if shared else "c5p"]
    M = tau.ffi.select_tile_rows(T, E + shared, K + shared, real_h, real_i)
    res = run(bins, "base", x, logits, gu, dn, K, M, 0, shared=shared)
    ids, w = oracle.route(logits[:, :E], K)
    r = res["routes"]
    np.testing.assert_array_equal(r[:, :K].astype(np.int64), ids)
    np.testing.assert_array_equal(r[:, K + shared:2 * K + shared], w)
    if shared:
        gate = oracle.sigmoid(logits[:, E])
        assert np.all(r[:, K] == E)
        np.testing.assert_array_equal(r[:, 2 * K + 1], gate)
        ids = np.concatenate([ids, np.full((T, 1), E, np.int64)], 1)
        w = np.concatenate([w, gate[:, None]], 1).astype(np.float32)
    meta, offsets, slots, tiles = oracle.dispatch(ids, E + shared, M, res["cap"])
    for key, ref in (("meta", meta), ("offsets", offsets), ("slots", slots), ("tiles", tiles)):
        np.testing.assert_array_equal(res[key], ref, err_msg=key)
    ref = oracle.moe(x, ids, w, gu, dn, bf16=True)
    got = from_bits(res["output"])
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 2e-3
    if shared:  # Zipf routing: most blocks hold a few rows, the 32-row split's case
        counts = meta[:E]
        assert ((counts > 0) & (counts <= 32)).sum() > (counts > 0).sum() // 2
        split = run(bins, "split32", x, logits, gu, dn, K, M, 0, shared=shared)
        for key in ("routes", "slots", "contributions", "output"):
            np.testing.assert_array_equal(split[key], res[key], err_msg=key)


def test_issued_mfma_work_matches_the_plan(bins, oracle):
    """The MFMA work the 256-row tiles issue, counted in the emulator, equals
    what the dispatch plan implies, on c3's token, expert and top-k counts with
    its N(0,1) router bias (hidden = intermediate = 64 keep it cheap; one
    64-deep K step and one column tile per projection):
      * shipped 4x4 waves (64x64 wave tiles): a wave runs its 16 MFMAs per K
        step unless its 64 rows are all padding -> 64 * ceil(live/64) per block;
      * -DTAU_FRAG_SKIP and the 128x128 wave tiles: MFMAs only for 32-row
        fragments holding a live row -> 32 * ceil(live/32) per block;
      * the 128x128 wave tiles without the skip: 256 per block.
    At these sizes useful work is one MFMA per assignment per projection, so
    the ratios are the padding overheads quoted for c3 (about 1.14x, 1.07x and
    1.63x).  The operand copies are counted too: every build stages the whole
    weight panel and skips A's all-padding 8-row groups."""
    T, E, K, H, I = 4096, 128, 8, 64, 64
    rng = np.random.default_rng(2)
    x = from_bits(bf16_bits(rng.standard_normal((T, H))))
    gu = from_bits(bf16_bits(rng.standard_normal((E, 2 * I, H)) * 0.05))
    dn = from_bits(bf16_bits(rng.standard_normal((E, H, I)) * 0.05))
    logits = rng.standard_normal((T, E)).astype(np.float32) + rng.standard_normal(E).astype(np.float32)
    logits = from_bits(bf16_bits(logits))
    import concurrent.futures
    builds = ("base", "fragskip", "bigwaves", "bigwaves_noskip")
    with concurrent.futures.ThreadPoolExecutor(4) as ex:
        futs = {v: ex.submit(run, bins, v, x, logits, gu, dn, K, 256, 0) for v in builds}
        res = {v: f.result() for v, f in futs.items()}
    counts = res["base"]["meta"][:E]
    lives = [min(256, n - b) for n in counts for b in range(0, n, 256)]
    per_block = {"base": lambda l: 64 * -(-l // 64), "fragskip": lambda l: 32 * -(-l // 32),
                 "bigwaves": lambda l: 32 * -(-l // 32), "bigwaves_noskip": lambda l: 256}
    projections = 2  # gate_up and down: one K step and one column tile each at these sizes
    for v in builds:
        expected = projections * sum(per_block[v](l) for l in lives)
        assert res[v]["counts"]["mfma32"] == expected, (v, res[v]["counts"], expected)
        assert res[v]["counts"]["mfma16"] == 0
        # direct-to-LDS copies (1 KB per wave instruction): per block and K step
        # the 256x64 weight panel (32) and the A rows in 8-row groups, all-padding
        # groups skipped (ceil(live/8))
        assert res[v]["counts"]["dma16"] == projections * sum(32 + -(-l // 8) for l in lives), v
        np.testing.assert_array_equal(res[v]["output"], res["base"]["output"], err_msg=v)
    useful = projections * T * K
    ratio = {v: res[v]["counts"]["mfma32"] / useful for v in builds}
    assert ratio["fragskip"] == ratio["bigwaves"] < ratio["base"] < ratio["bigwaves_noskip"]
    print("issued / useful MFMA rows:", {v: round(r, 3) for v, r in ratio.items()})
