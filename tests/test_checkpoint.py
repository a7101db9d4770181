"""Checkpoint loading of one sparse-MoE layer (host side; the GPU test is in
test_gpu_08_checkpoint.py).  Synthetic checkpoints in both of the reference's
expert layouts (tensors.rs:37-110) must assemble the same packed tensors, and
contract violations must name the offending tensor."""
import pytest
import torch
from safetensors.torch import save_file

E, H, I, IS = 4, 64, 32, 32
P = "model.layers.3"


def tensors(seed=0):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16)
    return {"router": r(E, H), "gate": r(E, I, H), "up": r(E, I, H), "down": r(E, H, I),
            "sg": r(IS, H), "su": r(IS, H), "sd": r(H, IS), "sgate": r(1, H)}


def shared_entries(t):
    return {f"{P}.mlp.shared_expert.gate_proj.weight": t["sg"], f"{P}.mlp.shared_expert.up_proj.weight": t["su"],
            f"{P}.mlp.shared_expert.down_proj.weight": t["sd"], f"{P}.mlp.shared_expert_gate.weight": t["sgate"]}


def write_individual(tmp_path, t):
    a = {f"{P}.mlp.gate.weight": t["router"]}
    b = dict(shared_entries(t))
    for e in range(E):
        d = a if e % 2 == 0 else b  # experts spread over two shards
        d[f"{P}.mlp.experts.{e}.gate_proj.weight"] = t["gate"][e].clone()
        d[f"{P}.mlp.experts.{e}.up_proj.weight"] = t["up"][e].clone()
        d[f"{P}.mlp.experts.{e}.down_proj.weight"] = t["down"][e].clone()
    pa, pb = str(tmp_path / "i-00001.safetensors"), str(tmp_path / "i-00002.safetensors")
    save_file(a, pa)
    save_file(b, pb)
    return [pa, pb]


def write_packed(tmp_path, t):
    d = {f"{P}.mlp.gate.weight": t["router"], f"{P}.mlp.experts.gate_up_proj": torch.cat([t["gate"], t["up"]], 1),
         f"{P}.mlp.experts.down_proj": t["down"].clone(), **shared_entries(t)}
    p = str(tmp_path / "packed.safetensors")
    save_file(d, p)
    return [p]


def config(tau):
    return tau.SparseMoeConfig(H, I, E, 2, shared_expert=tau.SharedExpertConfig(IS, gated=True))


def test_both_expert_layouts_assemble_the_same_tensors(tau, tmp_path):
    t = tensors()
    a = tau.checkpoint.read_sparse_moe_tensors(write_individual(tmp_path, t), P, config(tau), device="cpu")
    b = tau.checkpoint.read_sparse_moe_tensors(write_packed(tmp_path, t), P, config(tau), device="cpu")
    for k in ("router", "gate_up", "down", "shared_gate_up", "shared_down", "shared_gate"):
        assert torch.equal(a[k], b[k]), k
    assert torch.equal(a["gate_up"][:, :I], t["gate"]) and torch.equal(a["gate_up"][:, I:], t["up"])
    assert torch.equal(a["shared_gate_up"][:IS], t["sg"]) and torch.equal(a["shared_gate_up"][IS:], t["su"])
    assert torch.equal(a["down"], t["down"]) and torch.equal(a["router"], t["router"])


def test_contract_violations_name_the_tensor(tau, tmp_path):
    t = tensors()
    paths = write_packed(tmp_path, t)
    with pytest.raises(tau.checkpoint.CheckpointError, match=r"experts\.gate_up_proj has shape \[4, 64, 64\], expected \[4, 66, 64\]"):
        bad = tau.SparseMoeConfig(H, I + 1, E, 2, shared_expert=tau.SharedExpertConfig(IS))
        tau.checkpoint.read_sparse_moe_tensors(paths, P, bad, device="cpu")
    with pytest.raises(tau.checkpoint.CheckpointError, match=r"missing tensor model\.layers\.4\.mlp\.gate\.weight"):
        tau.checkpoint.read_sparse_moe_tensors(paths, "model.layers.4", config(tau), device="cpu")
    ind = write_individual(tmp_path, t)
    with pytest.raises(tau.checkpoint.CheckpointError, match="missing tensor"):
        tau.checkpoint.read_sparse_moe_tensors(ind[:1], P, config(tau), device="cpu")  # second shard absent
