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


def variants(tau):
    """Logit edge cases for the rows the gate_up waves rank from the logits:
    heavy ties (ids break them), FP32 logits, an expert count that is not a
    multiple of 8 (unvectorised row reads) with K > 16, and a non-finite row
    (the plan is marked invalid and every output element is NaN)."""
    MoeShape = tau.inputs.MoeShape
    return [
        ("ties_bf16", MoeShape("ties", 256, 128, 8, 128, 64, 11), "frag16", "ties", torch.bfloat16),
        ("ties_f32", MoeShape("ties32", 256, 128, 8, 128, 40, 12), "row_major", "ties", torch.float32),
        ("f32_logits", MoeShape("f32", 512, 64, 6, 192, 33, 13), "frag16", None, torch.float32),
        ("e60_k20", MoeShape("e60", 256, 60, 20, 128, 24, 14), "row_major", None, torch.bfloat16),
        ("e60_k20_f32", MoeShape("e60f", 256, 60, 20, 128, 24, 15), "frag16", "ties", torch.float32),
        ("e250_k3", MoeShape("e250", 256, 250, 3, 64, 64, 16), "frag16", None, torch.bfloat16),
        ("nan_row", MoeShape("nan", 256, 128, 8, 128, 8, 17), "frag16", "nan", torch.bfloat16),
        ("inf_row_f32", MoeShape("inf", 256, 32, 4, 64, 5, 18), "row_major", "inf", torch.float32),
    ]


@pytest.mark.parametrize("idx", range(6))
def test_decode_path_matches_general_path(tau, idx):
    name, shape, layout = cases(tau)[idx]
    if shape.experts > 256:  # the fused path takes E <= 256; E = 512 stays general
        import dataclasses
        shape = dataclasses.replace(shape, experts=256, shared_intermediate=0)
    say(f"[decode path] {name} T={shape.tokens} E={shape.experts} K={shape.top_k} {layout}")
    layer = tau.inputs.make_layer(shape)
    compare_paths(tau, shape, layer, layout)


@pytest.mark.parametrize("idx", range(8))
def test_decode_path_logit_edge_cases(tau, idx):
    name, shape, layout, edit, dtype = variants(tau)[idx]
    say(f"[decode path] {name} T={shape.tokens} E={shape.experts} K={shape.top_k} {layout} {dtype}")
    layer = tau.inputs.make_layer(shape)
    lg = layer["x"].float() @ layer["router"].t()
    if edit == "ties":  # a coarse grid: many equal logits per row
        lg = torch.round(lg * 4) / 4
    elif edit == "nan":
        lg[3, 5] = float("nan")
    elif edit == "inf":
        lg[2, 0] = float("inf")
    layer["logits"] = lg.to(dtype).contiguous()
    if edit == "ties":
        row = layer["logits"][0].float()
        assert len(torch.unique(row)) < shape.experts  # the grid really ties
    compare_paths(tau, shape, layer, layout)


def compare_paths(tau, shape, layer, layout):
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


@pytest.mark.parametrize("layout", ["frag16", "row_major"])
def test_decode_projection_entry_point_reproduces_the_step(tau, layout):
    """tau_launch_moe_decode_projection_ex launches exactly the fused decode
    path's gate_up and down kernels (the bench times them apart): run after a
    step on the same routes they rewrite activated, contributions and the plan
    with identical bits."""
    shape = tau.inputs.CONFIGS["c2_30b_a3b_decode"]
    say(f"[decode projection] c2 {layout}")
    layer = tau.inputs.make_layer(shape)
    cfg = tau.SparseMoeConfig(shape.hidden, shape.intermediate, shape.experts, shape.top_k)
    runner = tau.MoePrefillRunner(cfg, layer["gate_up"], layer["down"], weight_layout=layout)
    assert runner.tile_rows_for(shape.tokens) == 16
    runner.forward(layer["x"], layer["logits"])
    torch.cuda.synchronize()
    ws = runner._ws
    T, H, I, E, K = shape.tokens, shape.hidden, shape.intermediate, shape.experts, shape.top_k
    act = ws["activated"][: T * K * I].clone()
    con = ws["contributions"][: T * K * H].clone()
    plan = {k: ws[k].clone() for k in ("meta", "offsets", "slots", "tiles")}
    for k in ("activated", "contributions", "meta", "offsets", "slots", "tiles"):
        ws[k].fill_(-1 if ws[k].dtype == torch.int32 else 7)
    tau.ffi.decode_projection_ex(layer["x"], runner.gate_up, ws, ws["activated"], T, H, I, E, K, 0,
                                 weight_layout=runner.layout)
    tau.ffi.decode_projection_ex(ws["activated"], runner.down, ws, ws["contributions"], T, H, I, E, K, 1,
                                 weight_layout=runner.layout)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(ws["activated"][: T * K * I]), bits(act))
    np.testing.assert_array_equal(bits(ws["contributions"][: T * K * H]), bits(con))
    cap = ws["capacity"]
    np.testing.assert_array_equal(ws["meta"][: 2 * E + 2].cpu().numpy(), plan["meta"][: 2 * E + 2].cpu().numpy())
    np.testing.assert_array_equal(ws["offsets"][: E + 1].cpu().numpy(), plan["offsets"][: E + 1].cpu().numpy())
    np.testing.assert_array_equal(ws["slots"][:cap].cpu().numpy(), plan["slots"][:cap].cpu().numpy())
    np.testing.assert_array_equal(ws["tiles"][: cap // 16].cpu().numpy(), plan["tiles"][: cap // 16].cpu().numpy())
