"""The always-on shared expert folded into the routed schedule (run with -m gpu).

The shared expert runs as expert E: every token takes it at rank K with weight
sigmoid(x . w_s) (tau_launch_moe_routing_shared_ex), and the grouped
gate_up / down / combine handle E+1 experts and K+1 picks.  Checks: the
routed ranks equal the routing kernel's bit for bit and rank K is (E,
sigmoid(gate)); the folded layer matches the f32 oracle of the reference's
separate shared combine (shared_expert.rs:39-69) to the north-star tolerance,
the oracle's BF16 contract of the same schedule run as E+1 experts closely,
and the unfolded block within BF16 rounding; the block from hidden states
equals the block given its logits bit for bit.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)


def say(msg):
    print(msg, flush=True)


def f32(t):
    return t.detach().float().cpu().numpy()


def bits(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy()


def rel_l2(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("t,e,k,dtype", [(64, 128, 8, torch.float32), (37, 512, 10, torch.float32),
                                         (100, 60, 20, torch.bfloat16), (5, 16, 4, torch.bfloat16)])
def test_shared_routing_ranks(tau, oracle, t, e, k, dtype):
    say(f"[shared routing] T={t} E={e} K={k} {dtype}")
    g = torch.Generator(device="cuda").manual_seed(t + e)
    logits = (torch.randn(t, e + 1, generator=g, device="cuda") * 2).to(dtype)
    logits[3 % t, 1] = float("nan")  # a rejected row
    routes = torch.empty(t, 2 * (k + 1), dtype=torch.float32, device="cuda")
    tau.ffi.routing_shared_ex(logits, routes, e, k)
    ref = torch.empty(t, 2 * k, dtype=torch.float32, device="cuda")
    tau.ffi.routing_ex(logits[:, :e].contiguous(), ref, e, k)
    torch.cuda.synchronize()
    r, rr = f32(routes), f32(ref)
    np.testing.assert_array_equal(r[:, :k], rr[:, :k])                  # routed ids
    np.testing.assert_array_equal(r[:, k + 1: 2 * k + 1], rr[:, k:])    # routed weights
    bad = np.isnan(rr[:, 0])
    assert bad[3 % t]
    assert np.all(np.isnan(r[bad, k])) and np.all(np.isnan(r[bad, 2 * k + 1]))
    assert np.all(r[~bad, k] == e)
    gate = f32(logits[:, e]).astype(np.float64)
    sig = 1.0 / (1.0 + np.exp(-gate))
    assert np.all(np.abs(r[~bad, 2 * k + 1] - sig[~bad]) <= 2e-7 + 2e-6 * sig[~bad])
    # bit for bit the f32 sigmoid of the reference's CPU path
    np.testing.assert_array_equal(r[~bad, 2 * k + 1], oracle.sigmoid(f32(logits[:, e]))[~bad])


def block_pair(tau, shape, router=False):
    layer = tau.inputs.make_layer(shape)
    cfg = tau.SparseMoeConfig(shape.hidden, shape.intermediate, shape.experts, shape.top_k,
                              shared_expert=tau.SharedExpertConfig(shape.shared_intermediate, gated=True))
    kw = {}
    if router:
        kw = dict(router_weight=layer["router"].to(torch.bfloat16), router_bias=layer["bias"])
    args = (cfg, layer["gate_up"], layer["down"], layer["shared_gate_up"], layer["shared_down"], layer["shared_gate"])
    folded = tau.SparseMoeBlock(*args, fold_shared=True, **kw)
    apart = tau.SparseMoeBlock(*args, fold_shared=False, **kw)
    return layer, folded, apart


@pytest.mark.parametrize("tokens", [8, 96, 600])
def test_folded_shared_expert_matches_oracle_and_unfolded_block(tau, oracle, tokens):
    shape = tau.inputs.scaled(tau.inputs.CONFIGS["c4_next_sparse"], tokens)
    say(f"[shared folded] T={tokens}")
    layer, folded, apart = block_pair(tau, shape)
    assert folded.folded and not apart.folded
    out = folded.forward(layer["x"], layer["logits"]).clone()
    ref_blk = apart.forward(layer["x"], layer["logits"])
    torch.cuda.synchronize()
    x = f32(layer["x"])
    K, E = shape.top_k, shape.experts
    ids, w = oracle.route(f32(layer["logits"]), K)
    routed32 = oracle.moe(x, ids, w, f32(layer["gate_up"]), f32(layer["down"]))
    sh32 = oracle.dense_mlp(x, f32(layer["shared_gate_up"]), f32(layer["shared_down"]))
    ref32 = oracle.shared_combine_f32(x, f32(layer["shared_gate"]), sh32, routed32)
    e32 = rel_l2(f32(out), ref32)
    e_blk = rel_l2(f32(out), f32(ref_blk))
    # the folded schedule's own BF16 contract: E+1 experts, rank K = (E, sigmoid(x . w_s))
    gate = x @ f32(layer["shared_gate"]).reshape(-1)
    ids1 = np.concatenate([ids, np.full((tokens, 1), E, ids.dtype)], 1)
    w1 = np.concatenate([w, (1.0 / (1.0 + np.exp(-gate.astype(np.float64)))).astype(np.float32)[:, None]], 1)
    gu1 = np.concatenate([f32(layer["gate_up"]), f32(layer["shared_gate_up"])[None]], 0)
    dn1 = np.concatenate([f32(layer["down"]), f32(layer["shared_down"])[None]], 0)
    ref16 = oracle.moe(x, ids1, w1, gu1, dn1, bf16=True)
    e16 = rel_l2(f32(out), ref16)
    say(f"    rel_l2 vs f32 {e32:.2e}, vs unfolded block {e_blk:.2e}, vs folded BF16 contract {e16:.2e}")
    assert e32 <= 1e-2
    assert e_blk <= 4e-3
    assert e16 <= 2e-3


@pytest.mark.parametrize("tokens", [40, 512])
def test_folded_block_from_hidden_states_equals_given_logits(tau, tokens):
    shape = tau.inputs.scaled(tau.inputs.CONFIGS["c4_next_sparse"], tokens)
    say(f"[shared folded router] T={tokens}")
    layer, folded, _ = block_pair(tau, shape, router=True)
    out = folded.forward(layer["x"]).clone()
    ext = folded._logits[:tokens].clone()  # [T, E+1]: router logits, then x . w_s
    given = folded.forward(layer["x"], ext).clone()
    given_e = folded.forward(layer["x"], ext[:, : shape.experts].contiguous())  # gate column projected apart
    torch.cuda.synchronize()
    assert ext.shape == (tokens, shape.experts + 1)
    np.testing.assert_array_equal(bits(out), bits(given))
    np.testing.assert_array_equal(bits(out), bits(given_e))
