"""The fused decode path (tau_launch_moe_prefill_ex with 16-row blocks and at
most 64 tokens) against the general path run as separate launches (dispatch,
grouped gate_up, grouped down, combine) on the same inputs: the outputs must
be bit-identical (same MFMA sequence and roundings per element), and the plan
the decode path builds inside its down launch must equal the dispatch kernel's
(run with -m gpu)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)


def say(msg):
    print(msg, flush=True)


def bits(t):
    return t.detach().view(torch.int16).cpu().numpy()


def cases(tau):
    C = tau.inputs.CONFIGS
    S = tau.inputs.scaled
    return [
        ("c2", C["c2_30b_a3b_decode"], "frag16"),
        ("c2", C["c2_30b_a3b_decode"], "row_major"),
        ("c5d", C["c5_235b_decode"], "frag16"),
        ("c2_t1", S(C["c2_30b_a3b_decode"], 1), "frag16"),
        ("c2_t17", S(C["c2_30b_a3b_decode"], 17), "row_major"),
        ("c4_t48", S(C["c4_next_sparse"], 48), "frag16"),
    ]


@pytest.mark.parametrize("idx", range(6))
def test_decode_path_matches_general_path(tau, idx):
    name, shape, layout = cases(tau)[idx]
    if shape.experts > 256:  # the fused path takes E <= 256; E = 512 stays general
        import dataclasses
        shape = dataclasses.replace(shape, experts=256, shared_intermediate=0)
    say(f"[decode path] {name} T={shape.tokens} E={shape.experts} K={shape.top_k} {layout}")
    layer = tau.inputs.make_layer(shape)
    T, H, I, E, K = shape.tokens, shape.hidden, shape.intermediate, shape.experts, shape.top_k
    cfg = tau.SparseMoeConfig(H, I, E, K)
    runner = tau.MoePrefillRunner(cfg, layer["gate_up"], layer["down"], 16, weight_layout=layout)
    fused = runner.forward(layer["x"], layer["logits"])
    torch.cuda.synchronize()
    v = {k: t.clone() for k, t in runner.plan_views(T).items()}

    ffi = tau.ffi
    ws = runner.workspace(T, 16)
    cap = ws["capacity"]
    routes = torch.empty(T * 2 * K, dtype=torch.float32, device="cuda")
    meta = torch.empty(2 * E + 2, dtype=torch.int32, device="cuda")
    offsets = torch.empty(E + 1, dtype=torch.int32, device="cuda")
    slots = torch.empty(cap, dtype=torch.int32, device="cuda")
    tiles = torch.empty(cap // 16, dtype=torch.int32, device="cuda")
    act = torch.zeros(cap * I, dtype=torch.bfloat16, device="cuda")
    contrib = torch.zeros(T * K * H, dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(layer["x"])
    g = {"routes": routes, "slots": slots, "tiles": tiles, "meta": meta, "capacity": cap}
    ffi.dispatch_ex(layer["logits"], routes, meta, offsets, slots, tiles, T, E, K, 16, cap)
    ffi.grouped_gemm_ex(layer["x"], runner.gate_up, g, act, T, H, I, E, K, 16, 0, weight_layout=runner.layout)
    ffi.grouped_gemm_ex(act, runner.down, g, contrib, T, H, I, E, K, 16, 1, weight_layout=runner.layout)
    ffi.combine_ex(contrib, out, meta, T, H, E, K)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(fused), bits(out))
    np.testing.assert_array_equal(v["routes"].cpu().numpy().ravel(), routes.cpu().numpy())
    np.testing.assert_array_equal(v["meta"].cpu().numpy(), meta.cpu().numpy())
    np.testing.assert_array_equal(v["offsets"].cpu().numpy(), offsets.cpu().numpy())
    np.testing.assert_array_equal(v["slots"].cpu().numpy()[:cap], slots.cpu().numpy())
    np.testing.assert_array_equal(v["tiles"].cpu().numpy()[: cap // 16], tiles.cpu().numpy())
