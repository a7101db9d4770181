"""FRAG16 weights on the GPU (run with -m gpu).

tau_moe_pack_weights must reproduce the header's fragment order exactly
(checked against the host restatement in frag16_host.py), and a layer run on
FRAG16 weights must be bit-identical to the same layer on row-major weights:
both layouts feed the same operand fragments to the same MFMA sequence in the
same K order, so any difference is an indexing error, not rounding.
"""
import numpy as np
import pytest

from frag16_host import frag16_permute

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)


def say(msg):
    print(msg, flush=True)


def bits(t):
    return t.detach().view(torch.int16).cpu().numpy()


@pytest.mark.parametrize("shape", [(3, 48, 128), (64, 192), (2, 1536, 2048)])
def test_pack_matches_header_order(tau, shape):
    say(f"[frag16 pack] {shape}")
    g = torch.Generator(device="cuda").manual_seed(11)
    w = torch.randn(shape, generator=g, device="cuda").to(torch.bfloat16)
    packed = tau.ffi.pack_weights(w)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(packed), frag16_permute(bits(w)))


def layer_shapes(tau):
    C = tau.inputs.CONFIGS
    S = tau.inputs.scaled
    return [
        ("c1_bf16", tau.inputs.MoeShape("c1_bf16", 256, 8, 2, 512, 16, 0)),
        ("c2", C["c2_30b_a3b_decode"]),
        ("c3_t256", S(C["c3_30b_a3b_prefill"], 256)),
        ("c4_t128", S(C["c4_next_sparse"], 128)),
        ("c5d", C["c5_235b_decode"]),
    ]


@pytest.mark.parametrize("idx", range(5))
def test_frag16_layer_bit_identical_to_row_major(tau, idx):
    name, shape = layer_shapes(tau)[idx]
    layer = tau.inputs.make_layer(shape)
    cfg = tau.SparseMoeConfig(shape.hidden, shape.intermediate, shape.experts, shape.top_k)
    for tile_rows in (16, 32, 64, 128, 256):
        say(f"[frag16 layer] {name} T={shape.tokens} M={tile_rows}")
        rm = tau.MoePrefillRunner(cfg, layer["gate_up"], layer["down"], tile_rows, weight_layout="row_major")
        fr = tau.MoePrefillRunner(cfg, layer["gate_up"], layer["down"], tile_rows, weight_layout="frag16")
        assert fr.layout == tau.ffi.WEIGHTS_FRAG16 and rm.layout == tau.ffi.WEIGHTS_ROW_MAJOR
        a = rm.forward(layer["x"], layer["logits"])
        b = fr.forward(layer["x"], layer["logits"])
        torch.cuda.synchronize()
        # same row block (the streaming kernels pick other column/K batches for frag16)
        assert [r[0] for r in rm.executed_tiles()] == [r[0] for r in fr.executed_tiles()] == [tile_rows] * 2
        np.testing.assert_array_equal(bits(a), bits(b))
        del rm, fr


@pytest.mark.parametrize("projection", [0, 1])
def test_frag16_grouped_projection_bit_identical(tau, projection):
    shape = tau.inputs.scaled(tau.inputs.CONFIGS["c3_30b_a3b_prefill"], 512)
    say(f"[frag16 projection] {projection} T={shape.tokens}")
    layer = tau.inputs.make_layer(shape)
    cfg = tau.SparseMoeConfig(shape.hidden, shape.intermediate, shape.experts, shape.top_k)
    runner = tau.MoePrefillRunner(cfg, layer["gate_up"], layer["down"], 128, weight_layout="row_major")
    runner.forward(layer["x"], layer["logits"])  # routes, dispatch and activations in the workspace
    ws = runner._ws
    w_rm = layer["gate_up"] if projection == 0 else layer["down"]
    w_fr = tau.ffi.pack_weights(w_rm)
    a = layer["x"] if projection == 0 else ws["activated"]
    out_shape = ws["activated"] if projection == 0 else ws["contributions"]
    o1, o2 = torch.zeros_like(out_shape), torch.zeros_like(out_shape)  # dead tiles are not written
    for tile_rows in (128,):
        args = (shape.tokens, shape.hidden, shape.intermediate, shape.experts, shape.top_k, tile_rows, projection)
        tau.ffi.grouped_gemm_ex(a.clone(), w_rm, ws, o1, *args)
        tau.ffi.grouped_gemm_ex(a.clone(), w_fr, ws, o2, *args, weight_layout=tau.ffi.WEIGHTS_FRAG16)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(o1), bits(o2))


@pytest.mark.parametrize("fold", [False, True])
def test_frag16_shared_expert_bit_identical(tau, fold):
    shape = tau.inputs.scaled(tau.inputs.CONFIGS["c4_next_sparse"], 96)
    say(f"[frag16 shared expert] T={shape.tokens} folded={fold}")
    layer = tau.inputs.make_layer(shape)
    cfg = tau.SparseMoeConfig(shape.hidden, shape.intermediate, shape.experts, shape.top_k,
                              shared_expert=tau.SharedExpertConfig(shape.shared_intermediate, gated=True))
    outs = []
    for lay in ("row_major", "frag16"):
        blk = tau.SparseMoeBlock(cfg, layer["gate_up"], layer["down"], layer["shared_gate_up"],
                                 layer["shared_down"], layer["shared_gate"], weight_layout=lay, fold_shared=fold)
        outs.append(blk.forward(layer["x"], layer["logits"]))
        torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(outs[0]), bits(outs[1]))
