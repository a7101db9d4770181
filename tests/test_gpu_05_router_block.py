"""Router projection and the whole block from x (run with -m gpu).

tau_launch_moe_router_ex: logits = x . W_r^T (+ b) in f32 (routing.rs:91-93).
On dyadic operands every product and partial sum is exact in f32, so the GPU
logits must equal the oracle's f32 linear bit for bit; SparseMoeBlock.forward(x)
then routes those logits exactly as the oracle does and matches its layer
output to the north-star tolerance.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)


def say(msg):
    print(msg, flush=True)


def to_np(t):
    return t.detach().float().cpu().numpy()


def dyadic(shape, seed):
    n = int(np.prod(shape))
    v = (((np.arange(n) * 17 + seed) % 31).astype(np.float32) - 15.0) / 128.0
    return v.reshape(shape)


@pytest.mark.parametrize("t,h,e,bias", [(33, 144, 8, False), (7, 256, 128, True), (300, 256, 64, True)])
def test_router_projection_exact_on_dyadic_operands(tau, oracle, t, h, e, bias):
    say(f"[router] T={t} H={h} E={e} bias={bias}")
    x = dyadic((t, h), 3)
    w = dyadic((e, h), 5)
    b = (np.arange(e, dtype=np.float32) - e / 2) / 64.0 if bias else None
    xt = torch.tensor(x).to(torch.bfloat16).cuda()
    wt = torch.tensor(w).to(torch.bfloat16).cuda()
    bt = torch.tensor(b).cuda() if bias else None
    logits = torch.empty(t, e, dtype=torch.float32, device="cuda")
    tau.ffi.router_ex(xt, wt, bt, logits)
    torch.cuda.synchronize()
    ref = oracle.linear(x, w)
    if bias:
        ref = ref + b[None, :]
    np.testing.assert_array_equal(to_np(logits), ref)


def rel_l2(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("name", ["c2_30b_a3b_decode", "c3_30b_a3b_prefill"])
def test_block_forward_from_hidden_states(tau, oracle, name):
    shape = tau.inputs.CONFIGS[name]
    if shape.tokens > 256:
        shape = tau.inputs.scaled(shape, 256)
    say(f"[block from x] {shape.name}")
    layer = tau.inputs.make_layer(shape)
    w_r = layer["router"].to(torch.bfloat16)
    cfg = tau.SparseMoeConfig(shape.hidden, shape.intermediate, shape.experts, shape.top_k)
    blk = tau.SparseMoeBlock(cfg, layer["gate_up"], layer["down"], router_weight=w_r, router_bias=layer["bias"])
    out = blk.forward(layer["x"])
    torch.cuda.synchronize()
    x = to_np(layer["x"])
    logits = to_np(blk._logits[: shape.tokens])
    ref_logits = oracle.linear(x, to_np(w_r)) + to_np(layer["bias"])[None, :]
    err = np.abs(logits - ref_logits)
    assert np.all(err <= 1e-5 * np.abs(ref_logits) + 1e-5), float(err.max())  # f32 order differences only
    K = shape.top_k
    ids, w = oracle.route(logits, K)
    routes = to_np(blk.runner.plan_views(shape.tokens)["routes"])
    np.testing.assert_array_equal(routes[:, :K].astype(np.int64), ids)
    ref = oracle.moe(x, ids, w, to_np(layer["gate_up"]), to_np(layer["down"]))
    e = rel_l2(to_np(out), ref)
    say(f"    rel_l2 vs f32 oracle {e:.2e}")
    assert e <= 1e-2


@pytest.mark.parametrize("which", ["c2", "c3_t256", "c4_t96"])
def test_fused_residual_equals_separate_bf16_add(tau, which):
    """forward(x, residual=r) == bf16(f32(forward(x)) + f32(r)) bit for bit, on
    the fused decode path (c2), the general path (c3) and with the shared
    expert finishing the block (c4)."""
    C = tau.inputs.CONFIGS
    shape = {"c2": C["c2_30b_a3b_decode"], "c3_t256": tau.inputs.scaled(C["c3_30b_a3b_prefill"], 256),
             "c4_t96": tau.inputs.scaled(C["c4_next_sparse"], 96)}[which]
    say(f"[residual] {shape.name}")
    layer = tau.inputs.make_layer(shape)
    shared = None
    if shape.shared_intermediate:
        shared = tau.SharedExpertConfig(shape.shared_intermediate, gated=True)
    cfg = tau.SparseMoeConfig(shape.hidden, shape.intermediate, shape.experts, shape.top_k, shared_expert=shared)
    blk = tau.SparseMoeBlock(cfg, layer["gate_up"], layer["down"], layer.get("shared_gate_up"),
                             layer.get("shared_down"), layer.get("shared_gate"))
    g = torch.Generator(device="cuda").manual_seed(9)
    res = torch.randn(layer["x"].shape, generator=g, device="cuda").to(torch.bfloat16)
    plain = blk.forward(layer["x"], layer["logits"]).clone()
    fused = blk.forward(layer["x"], layer["logits"], residual=res)
    torch.cuda.synchronize()
    expect = (plain.float() + res.float()).to(torch.bfloat16)
    np.testing.assert_array_equal(fused.view(torch.int16).cpu().numpy(), expect.view(torch.int16).cpu().numpy())


@pytest.mark.parametrize("t,h,e,k,bias", [(33, 160, 8, 2, False), (17, 96, 20, 4, True), (7, 256, 128, 8, True),
                                          (300, 256, 64, 6, True), (64, 2048, 128, 8, False),
                                          (40, 512, 512, 10, True), (5, 64, 256, 32, False)])
def test_fused_router_routing_exact_on_dyadic_operands(tau, oracle, t, h, e, k, bias):
    """tau_launch_moe_router_route_ex: the projection exact on dyadic operands,
    and the routes those logits give under the routing kernel and the oracle,
    bit for bit."""
    say(f"[fused router] T={t} H={h} E={e} K={k} bias={bias}")
    x = dyadic((t, h), 3)
    w = dyadic((e, h), 5)
    b = (np.arange(e, dtype=np.float32) - e / 2) / 64.0 if bias else None
    xt = torch.tensor(x).to(torch.bfloat16).cuda()
    wt = torch.tensor(w).to(torch.bfloat16).cuda()
    bt = torch.tensor(b).cuda() if bias else None
    logits = torch.empty(t, e, dtype=torch.float32, device="cuda")
    routes = torch.empty(t, 2 * k, dtype=torch.float32, device="cuda")
    tau.ffi.router_route_ex(xt, wt, bt, logits, routes, k)
    ref_routes = torch.empty_like(routes)
    tau.ffi.routing_ex(logits, ref_routes, e, k)
    torch.cuda.synchronize()
    ref = oracle.linear(x, w)
    if bias:
        ref = ref + b[None, :]
    np.testing.assert_array_equal(to_np(logits), ref)
    np.testing.assert_array_equal(to_np(routes), to_np(ref_routes))
    ids, _ = oracle.route(ref, k)
    np.testing.assert_array_equal(to_np(routes)[:, :k].astype(np.int64), ids)
    # the projection is router_ex's, bit for bit (same kernel for H % 32 == 0)
    logits2 = torch.empty_like(logits)
    tau.ffi.router_ex(xt, wt, bt, logits2)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_np(logits2), to_np(logits))


@pytest.mark.parametrize("name", ["c2_30b_a3b_decode", "c3_30b_a3b_prefill", "c5_235b_decode"])
def test_block_fused_router_equals_block_given_its_logits(tau, name):
    """forward(x) (router + routing call) == forward(x, logits) on the logits
    that call produced, bit for bit; the routes agree with the routing
    kernel's on those logits."""
    shape = tau.inputs.CONFIGS[name]
    if shape.tokens > 512:
        shape = tau.inputs.scaled(shape, 512)
    say(f"[fused router block] {shape.name}")
    layer = tau.inputs.make_layer(shape)
    cfg = tau.SparseMoeConfig(shape.hidden, shape.intermediate, shape.experts, shape.top_k)
    blk = tau.SparseMoeBlock(cfg, layer["gate_up"], layer["down"], router_weight=layer["router"].to(torch.bfloat16),
                             router_bias=layer["bias"])
    fused = blk.forward(layer["x"]).clone()
    logits = blk._logits[: shape.tokens].clone()
    routes = blk.runner.plan_views(shape.tokens)["routes"].clone()
    given = blk.forward(layer["x"], logits)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(fused.view(torch.int16).cpu().numpy(), given.view(torch.int16).cpu().numpy())
    np.testing.assert_array_equal(to_np(routes), to_np(blk.runner.plan_views(shape.tokens)["routes"]))


@pytest.mark.parametrize("t,h,e,k", [(9, 100, 8, 2), (33, 144, 20, 4)])
def test_router_routing_on_unaligned_hidden_sizes(tau, oracle, t, h, e, k):
    """H % 32 != 0 (and a misaligned input view): the projection falls back to
    the general linear kernel; still exact on dyadic operands."""
    say(f"[router fallback] T={t} H={h} E={e} K={k}")
    x = dyadic((t, h), 7)
    w = dyadic((e, h), 9)
    buf = torch.zeros(t * h + 8, dtype=torch.bfloat16, device="cuda")
    xt = buf[4: 4 + t * h].view(t, h)
    xt.copy_(torch.tensor(x).to(torch.bfloat16))
    wt = torch.tensor(w).to(torch.bfloat16).cuda()
    logits = torch.empty(t, e, dtype=torch.float32, device="cuda")
    routes = torch.empty(t, 2 * k, dtype=torch.float32, device="cuda")
    tau.ffi.router_route_ex(xt, wt, None, logits, routes, k)
    torch.cuda.synchronize()
    ref = oracle.linear(x, w)
    np.testing.assert_array_equal(to_np(logits), ref)
    ids, _ = oracle.route(ref, k)
    np.testing.assert_array_equal(to_np(routes)[:, :k].astype(np.int64), ids)


def test_router_routing_rejects_bad_arguments(tau):
    w = torch.zeros(8, 64, dtype=torch.bfloat16, device="cuda")
    logits = torch.empty(8, 8, dtype=torch.float32, device="cuda")
    routes = torch.empty(8, 18, dtype=torch.float32, device="cuda")
    with pytest.raises(tau.ffi.LaunchError):  # K > E
        tau.ffi.router_route_ex(w, w, None, logits, routes, 9)
    with pytest.raises(tau.ffi.LaunchError):  # no logits buffer
        tau.ffi.router_route_ex(w, w, None, None, routes, 2)


@pytest.mark.parametrize("which", ["c2", "c3_t512", "c4_t300"])
def test_block_is_deterministic_run_to_run(tau, which):
    """No atomics in any reduction, a stable plan and a fixed-order K-split
    router: repeated runs from hidden states are bit-identical (decode path,
    general path with 128-row tiles, folded shared expert)."""
    C = tau.inputs.CONFIGS
    shape = {"c2": C["c2_30b_a3b_decode"], "c3_t512": tau.inputs.scaled(C["c3_30b_a3b_prefill"], 512),
             "c4_t300": tau.inputs.scaled(C["c4_next_sparse"], 300)}[which]
    say(f"[determinism] {shape.name}")
    layer = tau.inputs.make_layer(shape)
    shared = tau.SharedExpertConfig(shape.shared_intermediate) if shape.shared_intermediate else None
    cfg = tau.SparseMoeConfig(shape.hidden, shape.intermediate, shape.experts, shape.top_k, shared_expert=shared)
    blk = tau.SparseMoeBlock(cfg, layer["gate_up"], layer["down"], layer.get("shared_gate_up"),
                             layer.get("shared_down"), layer.get("shared_gate"),
                             router_weight=layer["router"].to(torch.bfloat16), router_bias=layer["bias"])
    outs = [blk.forward(layer["x"]).clone() for _ in range(3)]
    torch.cuda.synchronize()
    for o in outs[1:]:
        np.testing.assert_array_equal(o.view(torch.int16).cpu().numpy(), outs[0].view(torch.int16).cpu().numpy())
