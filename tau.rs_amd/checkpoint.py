"""Safetensors loading of one sparse-MoE layer (the reference's tensor contract,
crates/models/src/qwen3_5_moe/tensors.rs:37-110, and expert-bank assembly,
crates/models/src/components/sparse_moe/experts.rs:22-89).

Two expert layouts exist in Qwen3.5-MoE checkpoints under `{layer}.mlp`:

* individual (causal-LM checkpoints): `experts.{e}.gate_proj.weight` [I, H],
  `experts.{e}.up_proj.weight` [I, H], `experts.{e}.down_proj.weight` [H, I];
* packed (conditional-generation checkpoints): `experts.gate_up_proj`
  [E, 2I, H] (gate rows first) and `experts.down_proj` [E, H, I].

Both are assembled into the packed device tensors the kernels take.  The
router is `gate.weight` [E, H]; the optional shared expert is
`shared_expert.{gate,up,down}_proj.weight` with its gate
`shared_expert_gate.weight` [1, H].  Tensors are read lazily, one at a time,
and copied straight to the target device, so host memory stays at one tensor.
"""
from __future__ import annotations

import os
from typing import Dict, Iterable, Optional, Sequence

import torch

from .sparse_moe import SparseMoeBlock, SparseMoeConfig


class CheckpointError(ValueError):
    """A required tensor is missing or has the wrong shape or dtype."""


class _Shards:
    """Lazy view over the tensors of several safetensors files."""

    def __init__(self, paths: Sequence[str]):
        from safetensors import safe_open

        self._files = []
        self._where: Dict[str, int] = {}
        for i, path in enumerate(paths):
            if not os.path.exists(path):
                raise CheckpointError(f"checkpoint shard not found: {path}")
            f = safe_open(path, framework="pt")
            self._files.append(f)
            for k in f.keys():
                self._where.setdefault(k, i)

    def has(self, name: str) -> bool:
        return name in self._where

    def shape(self, name: str):
        f = self._files[self._where[name]]
        return tuple(f.get_slice(name).get_shape())

    def get(self, name: str) -> torch.Tensor:
        return self._files[self._where[name]].get_tensor(name)


def _expect(shards: _Shards, name: str, shape: Iterable[int]) -> None:
    shape = tuple(shape)
    if not shards.has(name):
        raise CheckpointError(f"missing tensor {name} (expected shape {list(shape)})")
    got = shards.shape(name)
    if got != shape:
        raise CheckpointError(f"tensor {name} has shape {list(got)}, expected {list(shape)}")


def _load(shards: _Shards, name: str, device, dtype) -> torch.Tensor:
    t = shards.get(name)
    if t.dtype != dtype:
        if not t.dtype.is_floating_point:
            raise CheckpointError(f"tensor {name} has dtype {t.dtype}, expected a floating-point type")
        t = t.to(dtype)
    return t.to(device)


def read_sparse_moe_tensors(paths: Sequence[str], layer_prefix: str, config: SparseMoeConfig,
                            device="cuda", dtype=torch.bfloat16) -> Dict[str, torch.Tensor]:
    """Tensors of `{layer_prefix}.mlp`: router [E,H], gate_up [E,2I,H], down
    [E,H,I] and, when the config has a shared expert, shared_gate_up [2Is,H],
    shared_down [H,Is], shared_gate [1,H].  Shapes are checked before any
    tensor is read; the expert layout is detected from the names present."""
    config.validate()
    E, H, I = config.num_experts, config.hidden_size, config.expert_intermediate_size
    p = f"{layer_prefix}.mlp"
    shards = _Shards(paths)
    packed = shards.has(f"{p}.experts.gate_up_proj")
    _expect(shards, f"{p}.gate.weight", (E, H))
    if packed:
        _expect(shards, f"{p}.experts.gate_up_proj", (E, 2 * I, H))
        _expect(shards, f"{p}.experts.down_proj", (E, H, I))
    else:
        for e in range(E):
            _expect(shards, f"{p}.experts.{e}.gate_proj.weight", (I, H))
            _expect(shards, f"{p}.experts.{e}.up_proj.weight", (I, H))
            _expect(shards, f"{p}.experts.{e}.down_proj.weight", (H, I))
    se = config.shared_expert
    if se is not None:
        Is = se.intermediate_size
        _expect(shards, f"{p}.shared_expert.gate_proj.weight", (Is, H))
        _expect(shards, f"{p}.shared_expert.up_proj.weight", (Is, H))
        _expect(shards, f"{p}.shared_expert.down_proj.weight", (H, Is))
        if se.gated:
            _expect(shards, f"{p}.shared_expert_gate.weight", (1, H))

    out = {"router": _load(shards, f"{p}.gate.weight", device, dtype)}
    if packed:
        out["gate_up"] = _load(shards, f"{p}.experts.gate_up_proj", device, dtype).contiguous()
        out["down"] = _load(shards, f"{p}.experts.down_proj", device, dtype).contiguous()
    else:
        gate_up = torch.empty(E, 2 * I, H, dtype=dtype, device=device)
        down = torch.empty(E, H, I, dtype=dtype, device=device)
        for e in range(E):
            gate_up[e, :I] = _load(shards, f"{p}.experts.{e}.gate_proj.weight", device, dtype)
            gate_up[e, I:] = _load(shards, f"{p}.experts.{e}.up_proj.weight", device, dtype)
            down[e] = _load(shards, f"{p}.experts.{e}.down_proj.weight", device, dtype)
        out["gate_up"], out["down"] = gate_up, down
    if se is not None:
        g = _load(shards, f"{p}.shared_expert.gate_proj.weight", device, dtype)
        u = _load(shards, f"{p}.shared_expert.up_proj.weight", device, dtype)
        out["shared_gate_up"] = torch.cat([g, u], dim=0).contiguous()
        out["shared_down"] = _load(shards, f"{p}.shared_expert.down_proj.weight", device, dtype).contiguous()
        if se.gated:
            out["shared_gate"] = _load(shards, f"{p}.shared_expert_gate.weight", device, dtype).contiguous()
    return out


def load_sparse_moe_block(paths: Sequence[str], layer_prefix: str, config: SparseMoeConfig,
                          router_bias: Optional[torch.Tensor] = None, tile_rows: Optional[int] = None,
                          weight_layout: str = "auto") -> SparseMoeBlock:
    """A SparseMoeBlock on the GPU from a checkpoint layer (expert weights held
    in FRAG16 when the shape allows, see MoePrefillRunner)."""
    t = read_sparse_moe_tensors(paths, layer_prefix, config, device="cuda")
    return SparseMoeBlock(config, t["gate_up"], t["down"], t.get("shared_gate_up"), t.get("shared_down"),
                          t.get("shared_gate"), tile_rows=tile_rows, weight_layout=weight_layout,
                          router_weight=t["router"], router_bias=router_bias)
