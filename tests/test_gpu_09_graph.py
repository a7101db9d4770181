"""HIP-graph capture of the block (run with -m gpu): every replay, with fresh
inputs copied into the static buffers and eager work plus synchronisations in
between, equals an eager forward bit for bit."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)


def bits(t):
    return t.view(torch.int16).cpu().numpy()


@pytest.mark.parametrize("which", ["c2", "c3_t256", "c4_t96", "c4_t96_apart"])
def test_graph_replays_equal_eager(tau, which):
    C = tau.inputs.CONFIGS
    shape = {"c2": C["c2_30b_a3b_decode"], "c3_t256": tau.inputs.scaled(C["c3_30b_a3b_prefill"], 256),
             "c4_t96": tau.inputs.scaled(C["c4_next_sparse"], 96),
             "c4_t96_apart": tau.inputs.scaled(C["c4_next_sparse"], 96)}[which]
    print(f"[graph] {shape.name}", flush=True)
    layer = tau.inputs.make_layer(shape)
    shared = tau.SharedExpertConfig(shape.shared_intermediate) if shape.shared_intermediate else None
    cfg = tau.SparseMoeConfig(shape.hidden, shape.intermediate, shape.experts, shape.top_k, shared_expert=shared)
    blk = tau.SparseMoeBlock(cfg, layer["gate_up"], layer["down"], layer.get("shared_gate_up"),
                             layer.get("shared_down"), layer.get("shared_gate"),
                             router_weight=layer["router"].to(torch.bfloat16), router_bias=layer["bias"],
                             fold_shared=False if which.endswith("apart") else None)
    x = layer["x"].clone()
    res = torch.zeros_like(x) if shared is not None else None
    graph, out = blk.capture(x, None, residual=res)
    g = torch.Generator(device="cuda").manual_seed(4)
    for replay in range(4):
        x.copy_(torch.randn(x.shape, generator=g, device="cuda").to(torch.bfloat16))
        if res is not None:
            res.copy_(torch.randn(x.shape, generator=g, device="cuda").to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        got = bits(out)
        _ = (x.float() * 2).sum().item()  # eager work between replays
        eager = blk.forward(x.clone(), residual=None if res is None else res.clone())
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got, bits(eager), err_msg=f"replay {replay}")
