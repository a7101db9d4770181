"""Centered RMSNorm and the fused residual add + norm in front of the MoE block
(run with -m gpu).

Cases follow the reference's norm tests (crates/models/src/components/cuda/
rms_norm/tests/residual/correctness.rs and support.rs): the residual is exact
(storage-dtype sum), the normalized output is within one BF16 ulp (f32:
1e-6 + 2e-6|b|) of the f32 CPU oracle and of the f64 closed form, the fused
output equals the standalone norm of the residual bit for bit, inputs are not
modified, and results do not depend on the access-width policy or on pointer
alignment.  The decoder's feed-forward half (residual + norm, MoE block, final
residual add fused into the block) equals the separate steps bit for bit.
"""
import numpy as np
import pytest

from norm_host import assert_close, f64_norm, patterned

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)


def say(msg):
    print(msg, flush=True)


def dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dtype).cuda()


def host(t):
    return t.detach().float().cpu().numpy()


def bits(t):
    return t.detach().contiguous().view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32).cpu().numpy()


DTYPES = [torch.float32, torch.bfloat16]


def run_case(tau, oracle, rows, columns, dtype, policy=16, offsets=(0, 0, 0), eps=1e-6):
    """The reference's check(): patterned inputs in views that start `offsets`
    elements into their buffers (same values whatever the offset)."""
    bf16 = dtype == torch.bfloat16
    n = rows * columns
    def placed(values, offset):  # the same values at an element offset into a larger buffer
        buf = np.full(values.size + offset + 1, 7.0, np.float32)
        buf[offset: offset + values.size] = values
        return dev(buf, dtype)

    xs = placed(patterned(n, 3), offsets[0])
    bs = placed(patterned(n, 19), offsets[1])
    ws = placed(patterned(columns, 47), offsets[2])
    snap = [bits(xs), bits(bs), bits(ws)]
    x = xs[offsets[0]: offsets[0] + n].view(rows, columns)
    b = bs[offsets[1]: offsets[1] + n].view(rows, columns)
    w = ws[offsets[2]: offsets[2] + columns]
    res, y = tau.ffi.fused_residual_rms_norm(x, b, w, eps, preferred_bytes=policy)
    alone = tau.ffi.centered_rms_norm(res, w, eps, preferred_bytes=policy)
    torch.cuda.synchronize()
    ref_res, ref_y = oracle.centered_rms_norm(host(x), host(w), eps, branch=host(b), bf16=bf16)
    np.testing.assert_array_equal(host(res), ref_res)                 # storage-dtype sum: exact
    assert_close(host(y), f64_norm(ref_res, host(w), eps), bf16)      # f64 closed form
    if columns <= 5120:  # the reference's widths: within its bound of the f32 CPU path too
        assert_close(host(y), ref_y, bf16)
    else:  # the CPU path's sequential f32 sum drifts ~sqrt(columns) * 2^-24 from f64
        bound = 1e-6 + (2e-6 + 4 * np.sqrt(columns) * 2.0 ** -24) * np.abs(ref_y)
        assert np.all(np.abs(host(y) - ref_y) <= bound + (np.abs(ref_y) * 2.0 ** -7 if bf16 else 0))
    np.testing.assert_array_equal(bits(y), bits(alone))               # fused == norm(residual)
    for before, t in zip(snap, (xs, bs, ws)):                         # inputs untouched
        np.testing.assert_array_equal(before, bits(t))
    return res, y


@pytest.mark.parametrize("dtype", DTYPES)
def test_norm_decode_prefill_and_irregular_widths(tau, oracle, dtype):
    for columns in [1, 31, 32, 33, 255, 256, 257, 2560, 5120]:
        for rows in [1, 5]:
            say(f"[norm] {dtype} rows={rows} columns={columns}")
            run_case(tau, oracle, rows, columns, dtype)
    for columns in [2560, 5120]:
        say(f"[norm] {dtype} rows=512 columns={columns}")
        run_case(tau, oracle, 512, columns, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_norm_wide_rows_recompute_path(tau, oracle, dtype):
    # more than 16 chunks of 16 bytes per lane: the residual is recomputed in pass 2
    for columns in [9000, 20000]:
        say(f"[norm wide] {dtype} columns={columns}")
        run_case(tau, oracle, 3, columns, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_norm_policies_and_offsets_give_identical_bits(tau, oracle, dtype):
    for columns in [256, 2560, 5120]:
        say(f"[norm policy/offset] {dtype} columns={columns}")
        base_res, base_y = run_case(tau, oracle, 3, columns, dtype)
        for policy in [0, 4, 8, 16]:
            r, y = run_case(tau, oracle, 3, columns, dtype, policy=policy)
            np.testing.assert_array_equal(bits(r), bits(base_res))
            np.testing.assert_array_equal(bits(y), bits(base_y))
        for offsets in [(1, 0, 0), (0, 1, 0), (0, 0, 1), (2, 2, 2), (4, 4, 4), (8, 8, 8)]:
            r, y = run_case(tau, oracle, 3, columns, dtype, offsets=offsets)
            np.testing.assert_array_equal(bits(r), bits(base_res))
            np.testing.assert_array_equal(bits(y), bits(base_y))


def test_norm_rounds_bf16_sum_before_normalization_and_allows_aliases(tau, oracle):
    """residual/correctness.rs:43-91: the BF16 sum is rounded before the norm
    (expected sums worked by hand in test_oracle), and branch may alias input."""
    xin = np.array([1.0, 1.0, -1.0, 0.0, 1024.0, 0.0001, -0.0001, 1e4], np.float32)
    bin_ = np.array([0.00390625, 0.01171875, -0.00390625, 0.0, -1024.0, -0.00005, 0.00005, -9990.0], np.float32)
    r5 = 1.640625 * 2.0 ** -15
    expect = np.array([1.0, 1.015625, -1.0, 0.0, 0.0, r5, -r5, 0.0], np.float32)
    x = dev(np.tile(xin, 320), torch.bfloat16).view(1, 2560)
    b = dev(np.tile(bin_, 320), torch.bfloat16).view(1, 2560)
    w = dev(np.tile(np.array([0.0, -1.0, -1.5, 0.25], np.float32), 640), torch.bfloat16)
    for eps in (1e-6, 1e-3):
        say(f"[norm rounding] eps={eps}")
        res, y = tau.ffi.fused_residual_rms_norm(x, b, w, eps)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(res).reshape(-1, 8), np.tile(expect, (320, 1)))
        assert np.all(host(y).reshape(-1, 4)[:, 1] == 0.0)
        np.testing.assert_array_equal(bits(y), bits(tau.ffi.centered_rms_norm(res, w, eps)))
        _, ref_y = oracle.centered_rms_norm(host(x), host(w), eps, branch=host(b), bf16=True)
        assert_close(host(y), ref_y, True)
        # branch aliasing the input: residual = 2x, rounded
        res2, y2 = tau.ffi.fused_residual_rms_norm(x, x, w, eps)
        torch.cuda.synchronize()
        ref_res2, ref_y2 = oracle.centered_rms_norm(host(x), host(w), eps, branch=host(x), bf16=True)
        np.testing.assert_array_equal(host(res2), ref_res2)
        assert_close(host(y2), ref_y2, True)


def test_norm_rejects_invalid_contracts(tau):
    x = torch.zeros(2, 64, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(64, dtype=torch.bfloat16, device="cuda")
    L = tau.ffi.lib()
    s = tau.ffi.stream_ptr()
    p = tau.ffi.ptr
    ok = L.tau_launch_fused_residual_rms_norm(p(x), p(x), p(w), p(torch.empty_like(x)), p(torch.empty_like(x)),
                                              2, 64, 1e-6, 1, s, 16)
    assert ok == 0
    bad = [
        (p(x), p(x), p(w), p(x), p(x), 2, 64, 0.0, 1, s, 16),             # epsilon must be positive
        (p(x), p(x), p(w), p(x), p(x), 2, 64, float("inf"), 1, s, 16),    # and finite
        (p(x), p(x), p(w), p(x), p(x), 0, 64, 1e-6, 1, s, 16),            # rows
        (p(x), p(x), p(w), p(x), p(x), 2, 0, 1e-6, 1, s, 16),             # columns
        (p(x), p(x), p(w), p(x), p(x), 2, 64, 1e-6, 2, s, 16),            # dtype
        (p(x), p(x), p(w), p(x), p(x), 2, 64, 1e-6, 1, s, 3),             # vector policy
        (p(x), None, p(w), p(x), p(x), 2, 64, 1e-6, 1, s, 16),            # branch
        (p(x), p(x), p(w), None, p(x), 2, 64, 1e-6, 1, s, 16),            # residual output
        (p(x), p(x), None, p(x), p(x), 2, 64, 1e-6, 1, s, 16),            # weight
    ]
    for args in bad:
        assert L.tau_launch_fused_residual_rms_norm(*args) != 0, args
    assert L.tau_launch_centered_rms_norm(p(x), p(w), p(x), 2, 64, -1.0, 1, s) != 0
    assert L.tau_launch_centered_rms_norm_configured(p(x), p(w), p(x), 2, 64, 1e-6, 1, s, 12) != 0
    torch.cuda.synchronize()


@pytest.mark.parametrize("which", ["c2", "c3_t256"])
def test_moe_feed_forward_equals_separate_steps(tau, which):
    """decoder.rs:95-116 after the token mixer: residual_sum + MoE(norm(residual_sum)),
    with the add fused into the block, against the three steps run separately."""
    C = tau.inputs.CONFIGS
    shape = {"c2": C["c2_30b_a3b_decode"], "c3_t256": tau.inputs.scaled(C["c3_30b_a3b_prefill"], 256)}[which]
    say(f"[moe feed-forward] {shape.name}")
    layer = tau.inputs.make_layer(shape)
    H = shape.hidden
    cfg = tau.SparseMoeConfig(H, shape.intermediate, shape.experts, shape.top_k)
    blk = tau.SparseMoeBlock(cfg, layer["gate_up"], layer["down"], router_weight=layer["router"].to(torch.bfloat16),
                             router_bias=layer["bias"])
    g = torch.Generator(device="cuda").manual_seed(21)
    xs = torch.randn(layer["x"].shape, generator=g, device="cuda").to(torch.bfloat16)
    branch = torch.randn(layer["x"].shape, generator=g, device="cuda").to(torch.bfloat16)
    norm = tau.CenteredRmsNorm((torch.randn(H, generator=g, device="cuda") * 0.1).to(torch.bfloat16), 1e-6)
    out = tau.moe_feed_forward(xs, branch, norm, blk).clone()
    res, normalized = norm.add_residual_and_normalize(xs, branch)
    moe = blk.forward(normalized).clone()
    torch.cuda.synchronize()
    expect = (moe.float() + res.float()).to(torch.bfloat16)
    np.testing.assert_array_equal(bits(out), bits(expect))
    np.testing.assert_array_equal(bits(res), bits((xs.float() + branch.float()).to(torch.bfloat16)))
