"""CPU checks that pin the oracle (oracle/moe_oracle.c) before it is trusted.

Every check is independent of the oracle's own formulas: golden vectors the
reference ships, its closed-form unit tests, library routines (torch) for the
special cases the MoE reduces to, brute-force f64 sums, and invariants.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def load_router_fixture():
    from safetensors.numpy import load_file
    return load_file(os.path.join(GOLDEN, "moe_router_sm90.safetensors"))


# --- routing: golden vectors (crates/models/src/components/cuda/routing.rs:99-160)

def test_router_matches_sglang_golden_rows():
    d = load_router_fixture()
    scores, ids_ref, w_ref = d["scores"], d["ids"].astype(np.int64), d["weights"]
    ids, w = O.route(scores, 8)
    np.testing.assert_array_equal(ids, ids_ref)
    assert np.all(np.abs(w - w_ref) <= 1e-7 + 1e-5 * np.abs(w_ref))
    # Both within the f32 budget of an independent f64 selected softmax.
    for row in range(scores.shape[0]):
        sel = scores[row, ids_ref[row]].astype(np.float64)
        ex = np.exp(sel - sel[0])
        f64 = ex / ex.sum()
        assert np.all(np.abs(w[row] - f64) <= 1e-7 + 1e-5 * np.abs(f64))


def test_router_fixture_has_eighth_slot_ties_resolved_to_lower_id():
    d = load_router_fixture()
    scores, ids_ref = d["scores"], d["ids"].astype(np.int64)
    ties = 0
    for row in range(scores.shape[0]):
        eighth = scores[row, ids_ref[row, 7]]
        tied = np.nonzero(scores[row] == eighth)[0]
        outside = [e for e in tied if e not in ids_ref[row]]
        if outside:  # a tie across the selection boundary
            ties += 1
            assert all(e > ids_ref[row, 7] for e in outside)
    assert ties == 3  # moe_router_sm90.json: "eighth_slot_tie_rows": 3


# --- select_experts closed forms (crates/models/src/components/sparse_moe/routing.rs:263-296)

def test_select_experts_tie_break_cases():
    scores = np.zeros(256, np.float32)
    for e, v in [(56, 9.), (65, 8.), (99, 7.), (177, 6.), (124, 5.), (132, 4.), (142, 3.), (2, 2.), (102, 2.)]:
        scores[e] = v
    assert O.select_experts(scores, 8) == [56, 65, 99, 177, 124, 132, 142, 2]
    assert O.select_experts(np.ones(256, np.float32), 8) == list(range(8))
    assert O.select_experts(np.array([1., 2., 2.], np.float32), 3) == [1, 2, 0]


def test_select_experts_rejects_nonfinite_and_bad_counts():
    assert O.select_experts(np.array([np.nan], np.float32), 1) is None
    assert O.select_experts(np.array([np.inf], np.float32), 1) is None
    assert O.select_experts(np.array([1.], np.float32), 0) is None
    assert O.select_experts(np.array([1.], np.float32), 2) is None
    with pytest.raises(ValueError):
        O.route(np.array([[0., np.nan]], np.float32), 1)


def test_uniform_logits_route_to_first_ids_with_equal_weights():
    ids, w = O.route(np.zeros((3, 256), np.float32), 8)
    assert (ids == np.arange(8)).all()
    assert (w == np.float32(0.125)).all()


def test_router_weight_on_feature_zero_closed_form():
    # crates/models/src/components/sparse_moe/tests/prepared.rs:33-36,136-141:
    # router row e = e/32 on feature 0 -> input[0] > 0 selects E-1..E-8.
    E, H = 256, 4
    router = np.zeros((E, H), np.float32)
    router[:, 0] = np.arange(E) / 32.
    x = np.array([[1., 0, 0, 0], [-1., 0, 0, 0], [0., 0, 0, 0]], np.float32)
    ids, _ = O.route(x @ router.T, 8)
    assert list(ids[0]) == list(range(E - 1, E - 9, -1))
    assert list(ids[1]) == list(range(8))
    assert list(ids[2]) == list(range(8))


def test_unnormalised_weights_are_the_softmax_probabilities():
    # normalize_selected_weights = false (sparse_moe/config.rs:45, routing.rs:198-202):
    # the weights are the selected probabilities themselves; torch's f32 softmax
    # (an independent implementation) agrees to f32 rounding, and the
    # normalised weights are exactly those divided by their rank-ordered sum.
    rng = np.random.default_rng(7)
    lg = rng.standard_normal((64, 48)).astype(np.float32) * 3
    ids, raw = O.route(lg, 6, normalize=False)
    ids_n, w_n = O.route(lg, 6)
    np.testing.assert_array_equal(ids, ids_n)
    probs = torch.softmax(torch.from_numpy(lg).double(), -1).numpy()
    sel = np.take_along_axis(probs, ids.astype(np.int64), 1)
    assert np.all(np.abs(raw - sel) <= 1e-6 * sel + 1e-12)  # f32 rounding of exp, sum and quotient
    for t in range(lg.shape[0]):
        total = np.float32(0)
        for r in range(6):
            total = np.float32(total + raw[t, r])
        np.testing.assert_array_equal(w_n[t], (raw[t] / total).astype(np.float32))
    _, raw_all = O.route(lg, 48, normalize=False)
    assert np.all(np.abs(raw_all.astype(np.float64).sum(1) - 1) < 1e-5)


def test_experts_rank_on_probabilities_so_collapsed_logits_tie_to_lower_id():
    # routing.rs:139-141,239-257 compare f32 probabilities, not logits: two
    # distinct logits whose exp(x - max) rounds to the same float are a tie,
    # which the lower id wins even when its logit is the smaller one.
    # exp(-2^-25) = 1 - 2^-25 is halfway between 1 - 2^-24 and 1 and rounds to 1.
    tiny = np.float32(2.0 ** -25)
    lg = np.array([[-tiny, 0.0, -4.0, -5.0],      # id 0 has the smaller logit
                   [0.0, -tiny, -4.0, -5.0],
                   [-5.0, -4.0, 0.0, -np.float32(2.0 ** -23)]], np.float32)
    ids, w, p = O.route(lg, 2, want_probabilities=True)
    assert p[0, 0] == p[0, 1] and p[1, 0] == p[1, 1]
    assert list(ids[0]) == [0, 1] and list(ids[1]) == [0, 1]
    assert w[0, 0] == w[0, 1] == np.float32(0.5)
    # a 2^-23 gap survives exp (1 - 2^-23 is a float): the larger logit leads
    assert p[2, 2] > p[2, 3] and list(ids[2]) == [2, 3]


def test_sigmoid_gate_matches_f64_and_closed_forms():
    v = np.concatenate([np.linspace(-30, 30, 2001), [0.0, -200.0, 200.0, -np.inf, np.inf]]).astype(np.float32)
    s = O.sigmoid(v)
    ref = 1.0 / (1.0 + np.exp(-v.astype(np.float64)))
    assert np.all(np.abs(s - ref) <= 3 * np.spacing(np.float32(ref)) + 1e-45)
    assert s[-5] == np.float32(0.5) and s[-4] == 0.0 and s[-3] == 1.0 and s[-2] == 0.0 and s[-1] == 1.0


# --- whole block closed form (crates/models/src/components/sparse_moe/tests/block.rs:4-72)

def test_block_closed_form_individual_and_packed():
    I2 = np.eye(2, dtype=np.float32)
    x = np.array([[1., 0.], [0., 1.]], np.float32)
    ids, w = O.route(x @ I2.T, 1)
    gate_up = np.stack([np.concatenate([I2, I2]), np.concatenate([I2, I2])])
    down = np.stack([I2, 2 * I2])
    routed = O.moe(x, ids, w, gate_up, down, act=O.ACT_RELU)
    shared = O.dense_mlp(x, np.concatenate([I2, I2]), I2, act=O.ACT_RELU)
    out = O.shared_combine_f32(x, np.zeros((1, 2), np.float32), shared, routed)
    assert out.tolist() == [[1.5, 0.0], [0.0, 2.5]]


# --- special cases that reduce to library routines (torch, f64)

def _swiglu_torch(x, gate_up, down):
    x = torch.tensor(x, dtype=torch.float64)
    gu = torch.tensor(gate_up, dtype=torch.float64)
    dn = torch.tensor(down, dtype=torch.float64)
    i = gu.shape[0] // 2
    g = x @ gu[:i].T
    u = x @ gu[i:].T
    return (torch.nn.functional.silu(g) * u) @ dn.T


def test_single_expert_is_a_dense_swiglu_mlp():
    rng = np.random.default_rng(0)
    T, H, I = 9, 40, 24
    x = rng.standard_normal((T, H)).astype(np.float32)
    gu = (rng.standard_normal((1, 2 * I, H)) * 0.1).astype(np.float32)
    dn = (rng.standard_normal((1, H, I)) * 0.1).astype(np.float32)
    ids, w = O.route(np.zeros((T, 1), np.float32), 1)
    out = O.moe(x, ids, w, gu, dn)
    ref = _swiglu_torch(x, gu[0], dn[0]).numpy()
    np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-5)


def test_all_experts_selected_is_the_softmax_mixture():
    rng = np.random.default_rng(1)
    T, H, I, E = 7, 32, 16, 5
    x = rng.standard_normal((T, H)).astype(np.float32)
    gu = (rng.standard_normal((E, 2 * I, H)) * 0.1).astype(np.float32)
    dn = (rng.standard_normal((E, H, I)) * 0.1).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    ids, w = O.route(logits, E)
    out = O.moe(x, ids, w, gu, dn)
    p = torch.softmax(torch.tensor(logits, dtype=torch.float64), dim=-1)
    ref = sum(p[:, e:e + 1] * _swiglu_torch(x, gu[e], dn[e]) for e in range(E)).numpy()
    np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-5)


def test_expert_relabeling_and_token_split_invariance():
    rng = np.random.default_rng(2)
    T, H, I, E, K = 12, 24, 8, 6, 2
    x = rng.standard_normal((T, H)).astype(np.float32)
    gu = (rng.standard_normal((E, 2 * I, H)) * 0.1).astype(np.float32)
    dn = (rng.standard_normal((E, H, I)) * 0.1).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    ids, w = O.route(logits, K)
    out = O.moe(x, ids, w, gu, dn)
    perm = rng.permutation(E)
    ids2, w2 = O.route(logits[:, perm], K)
    out2 = O.moe(x, ids2, w2, gu[perm], dn[perm])
    np.testing.assert_array_equal(perm[ids2], ids)
    np.testing.assert_allclose(out2, out, rtol=1e-6, atol=1e-7)
    half = O.moe(x[:5], ids[:5], w[:5], gu, dn)
    np.testing.assert_allclose(half, out[:5], rtol=0, atol=0)


def test_token_mask_reproduces_rows_exactly():
    rng = np.random.default_rng(3)
    T, H, I, E, K = 20, 16, 8, 4, 2
    x = rng.standard_normal((T, H)).astype(np.float32)
    gu = (rng.standard_normal((E, 2 * I, H)) * 0.1).astype(np.float32)
    dn = (rng.standard_normal((E, H, I)) * 0.1).astype(np.float32)
    ids, w = O.route(rng.standard_normal((T, E)).astype(np.float32), K)
    full = O.moe(x, ids, w, gu, dn)
    mask = np.zeros(T, np.uint8)
    mask[[0, 7, 19]] = 1
    part = O.moe(x, ids, w, gu, dn, token_mask=mask)
    np.testing.assert_array_equal(part[mask == 1], full[mask == 1])


def test_gate_and_up_halves_are_not_interchangeable():
    # silu(g) * u is not symmetric: swapping the packed halves must change the result.
    rng = np.random.default_rng(4)
    T, H, I = 3, 8, 4
    x = rng.standard_normal((T, H)).astype(np.float32)
    gu = rng.standard_normal((1, 2 * I, H)).astype(np.float32)
    dn = rng.standard_normal((1, H, I)).astype(np.float32)
    ids, w = O.route(np.zeros((T, 1), np.float32), 1)
    a = O.moe(x, ids, w, gu, dn)
    b = O.moe(x, ids, w, np.concatenate([gu[:, I:], gu[:, :I]], axis=1), dn)
    assert not np.allclose(a, b)
    np.testing.assert_allclose(a, _swiglu_torch(x, gu[0], dn[0]).numpy(), rtol=1e-4, atol=1e-5)


# --- BF16 contract pieces

def test_dyadic_linear_is_exact():
    # crates/models/src/components/cuda/linear.rs:117-172 operands.
    for rows, cols, inner in [(1, 1, 7), (3, 11, 16), (17, 19, 33), (5, 32, 64)]:
        data = lambda n, seed: np.array([((i * 7 + seed) % 15 - 7) / 16. for i in range(n)], np.float32)
        x = data(rows * inner, 3).reshape(rows, inner)
        wt = data(cols * inner, 5).reshape(cols, inner)
        got = O.linear(x, wt)
        ref = (x.astype(np.float64) @ wt.astype(np.float64).T).astype(np.float32)
        np.testing.assert_array_equal(got, ref)


def weight_before_round_case():
    """Two experts, ReLU MLPs: expert 0's down output is exactly 1 + 1/256 (a
    BF16 halfway case) and expert 1's is zero, so the routed output is
    bf16(bf16((1 + 1/256) * w0)) (linear.rs:176-206 of the reference)."""
    x = np.array([[1., 1.]], np.float32)
    gate_up = np.zeros((2, 4, 2), np.float32)
    gate_up[:, 0:2, 0] = 1.0  # gate rows read feature 0 -> g = 1
    gate_up[:, 2:4, 1] = 1.0  # up rows read feature 1 -> u = 1
    down = np.zeros((2, 2, 2), np.float32)
    down[0, 0] = [1.0, 1.0 / 256.0]
    logits = np.array([[math.log(9.0), 0.0]], np.float32)
    return x, logits, gate_up, down


def test_weight_applied_before_bf16_round():
    x, logits, gate_up, down = weight_before_round_case()
    ids, w = O.route(logits, 2)
    assert list(ids[0]) == [0, 1]
    out = O.moe(x, ids, w, gate_up, down, act=O.ACT_RELU, bf16=True)
    dot = np.float32(1 + 1 / 256)
    exact = O.bf16_round(np.float32(dot * w[0, 0]))
    early = O.bf16_round(O.bf16_round(dot) * O.bf16_round(w[0, 0]))
    assert exact != early
    assert out[0, 0] == exact


def test_silu_and_mul_fixed_vectors():
    # crates/models/src/components/cuda/silu_and_mul.rs:183-186
    v = np.array([[1.0, -2.0, 0.5, 3.0, 2.0, 0.25, -4.0, 1.5],
                  [-0.5, 4.0, -3.0, 2.0, 1.25, -2.0, 0.75, 0.5]], np.float32)
    t = torch.tensor(v, dtype=torch.float64)
    ref = (torch.nn.functional.silu(t[:, :4]) * t[:, 4:]).numpy()
    np.testing.assert_allclose(O.silu_and_mul(v), ref, atol=1e-5)
    np.testing.assert_allclose(O.silu_and_mul(v, bf16=True), ref, atol=5e-2)


def test_bf16_contract_close_to_f32_path():
    rng = np.random.default_rng(5)
    T, H, I, E, K = 16, 64, 32, 8, 2
    bf = O.bf16_round
    x = bf(rng.standard_normal((T, H)))
    gu = bf(rng.standard_normal((E, 2 * I, H)) * 0.05)
    dn = bf(rng.standard_normal((E, H, I)) * 0.05)
    ids, w = O.route(bf(rng.standard_normal((T, E))), K)
    a = O.moe(x, ids, w, gu, dn)
    b = O.moe(x, ids, w, gu, dn, bf16=True)
    assert np.array_equal(b, bf(b))
    assert np.linalg.norm(a - b) / np.linalg.norm(a) < 1e-2


# --- dispatch invariants (crates/models/src/components/cuda/fused_moe/prefill/tests.rs:43-127)

@pytest.mark.parametrize("M", [16, 32, 128])
def test_dispatch_invariants(M):
    E, K = 256, 8
    for tokens in [257, 1, 15, 16, 17, 31, 32, 33, 255, 256, 1]:
        for concentrated in (False, True):
            ids = np.array([[r if concentrated else (t * 8 + r) % 256 for r in range(K)] for t in range(tokens)])
            meta, off, slots, tiles = O.dispatch(ids, E, M)
            cap = len(slots)
            assert meta[2 * E] == 0
            assert meta[:E].sum() == tokens * K
            padded = meta[2 * E + 1]
            assert padded <= cap and off[E] == padded
            seen = np.zeros(tokens * K, bool)
            for e in range(E):
                assert (off[e + 1] - off[e]) % M == 0
                assert meta[e] == meta[E + e]
                prev = -1
                n = 0
                for row in range(off[e], off[e + 1]):
                    assert tiles[row // M] == e
                    s = slots[row]
                    if s < tokens * K:
                        assert not seen[s]
                        seen[s] = True
                        assert (s % 8 if concentrated else s % 256) == e
                        assert s > prev  # stable: token-ascending
                        prev = s
                        n += 1
                    else:
                        assert s == tokens * K
                assert n == meta[e]
            assert seen.all()
            assert (tiles[padded // M:] == -1).all()


def test_capacity_closed_form():
    # crates/models/src/components/cuda/fused_moe/prefill/tests.rs:123-128
    assert O.capacity(1, 256, 8, 16) == 128
    assert O.capacity(0, 256, 8, 16) == -1


def test_plan_matches_stable_sort():
    rng = np.random.default_rng(6)
    T, E, K = 50, 12, 3
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)])
    counts, off, slots = O.plan(ids, E)
    order = sorted(range(T * K), key=lambda a: (ids.reshape(-1)[a], a))
    assert list(slots) == order
    assert list(counts) == [int((ids == e).sum()) for e in range(E)]


@pytest.mark.parametrize("width", [2, 17, 2048])
def test_shared_combine_bf16_against_f64_scalar_gate(width):
    # crates/models/src/components/cuda/shared_expert.rs:126-176 vectors.
    inp = np.zeros((3, width), np.float32)
    inp[0, 0], inp[0, 1], inp[2, 0] = 1., 1. / 256., -4.
    weight = np.zeros(width, np.float32)
    weight[0] = 1.
    weight[1 % width] = 1.
    shared = O.bf16_round(np.array([((i % 13) - 6.) / 16. for i in range(3 * width)], np.float32)).reshape(3, width)
    routed = O.bf16_round(np.array([((i % 17) - 8.) / 32. for i in range(3 * width)], np.float32)).reshape(3, width)
    got = O.shared_combine_bf16(inp, weight, shared, routed)
    for row in range(3):
        dot = float((inp[row].astype(np.float64) * weight).sum())
        gate = np.float64(np.float32(1. / (1. + math.exp(-dot))))
        exp = O.bf16_round((gate * shared[row] + routed[row]).astype(np.float32))
        np.testing.assert_array_equal(got[row], exp)


from norm_host import assert_close, f64_norm, patterned, to_dtype  # noqa: E402


# --- centered RMSNorm with the residual add (rms_norm.rs:66-150; the reference's
# norm tests: cuda/rms_norm/tests/residual/{correctness,support}.rs and the f64
# oracle of cuda/rms_norm/test_support.rs:5-27)

@pytest.mark.parametrize("bf16", [False, True])
def test_norm_oracle_matches_f64_closed_form(bf16):
    eps = 1e-6
    for columns in [1, 31, 32, 33, 255, 256, 257, 2560, 5120]:
        for rows in [1, 5]:
            x = to_dtype(patterned(rows * columns, 3), bf16).reshape(rows, columns)
            b = to_dtype(patterned(rows * columns, 19), bf16).reshape(rows, columns)
            w = to_dtype(patterned(columns, 47), bf16)
            res, y = O.centered_rms_norm(x, w, eps, branch=b, bf16=bf16)
            # the residual is the storage-dtype sum (torch's rounding, not the oracle's)
            np.testing.assert_array_equal(res, to_dtype(x + b, bf16))
            assert_close(y, f64_norm(res, w, eps), bf16)
            _, y2 = O.centered_rms_norm(res, w, eps, bf16=bf16)
            np.testing.assert_array_equal(y, y2)  # fused == norm of the residual


def test_norm_oracle_bf16_residual_rounding_known_answers():
    """residual/correctness.rs:43-91 inputs; the BF16 sums worked by hand:
    1 + 2^-8 ties to 1 (even), 1 + 3*2^-8 ties to 1 + 2^-6 (even), 1024 - 1024 = 0,
    bf16(1e4) = bf16(9990) = 9984, bf16(1e-4) = 1.640625 * 2^-14 and
    bf16(5e-5) = 1.640625 * 2^-15, whose difference is exact."""
    xin = np.array([1.0, 1.0, -1.0, 0.0, 1024.0, 0.0001, -0.0001, 1e4], np.float32)
    bin_ = np.array([0.00390625, 0.01171875, -0.00390625, 0.0, -1024.0, -0.00005, 0.00005, -9990.0], np.float32)
    r5 = 1.640625 * 2.0 ** -15
    expect = np.array([1.0, 1.015625, -1.0, 0.0, 0.0, r5, -r5, 0.0], np.float32)
    x = np.tile(to_dtype(xin, True), 320).reshape(1, 2560)
    b = np.tile(to_dtype(bin_, True), 320).reshape(1, 2560)
    w = np.tile(to_dtype(np.array([0.0, -1.0, -1.5, 0.25], np.float32), True), 640)
    for eps in (1e-6, 1e-3):
        res, y = O.centered_rms_norm(x, w, eps, branch=b, bf16=True)
        np.testing.assert_array_equal(res.reshape(-1, 8), np.tile(expect, (320, 1)))
        assert np.all(y.reshape(-1, 4)[:, 1] == 0.0)  # weight -1: the centred scale is exactly zero
        assert_close(y, f64_norm(res, w, eps), True)


def test_norm_oracle_divides_by_width_and_centres_the_scale():
    # constant rows normalise to +-1 (mean of squares, not their sum)
    for c in (2.0, -3.0, 0.5):
        for cols in (4, 100, 2048):
            _, y = O.centered_rms_norm(np.full((1, cols), c, np.float32), np.zeros(cols, np.float32), 1e-12)
            assert np.allclose(y, math.copysign(1.0, c), rtol=0, atol=2e-6)
    # weight w scales by 1 + w
    x = patterned(64, 5).reshape(1, 64)
    _, y0 = O.centered_rms_norm(x, np.zeros(64, np.float32), 1e-6)
    _, y1 = O.centered_rms_norm(x, np.ones(64, np.float32), 1e-6)
    np.testing.assert_array_equal(y1, y0 * 2)
