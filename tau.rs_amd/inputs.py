"""Synthetic MoE-layer workloads of the benchmark configurations.

Weights ~ N(0, 0.02) in the reference's packed layouts (gate_up [E, 2I, H] with
gate rows first, down [E, H, I]; crates/models/src/components/sparse_moe/
experts.rs:50-89), activations ~ N(0, 1), router W_r [E, H] ~ N(0, 0.02).
Router logits are an input of the path (the reference's router Linear runs
before its MoE launcher): they are computed once here in f32, rounded to
BF16 for the BF16 configurations, and the same values feed the HIP path and
the oracle.  Draws come from torch's Philox generator seeded per config.
"""
from __future__ import annotations

import dataclasses
import math

import torch


@dataclasses.dataclass(frozen=True)
class MoeShape:
    name: str
    hidden: int
    experts: int
    top_k: int
    intermediate: int
    tokens: int
    seed: int
    dtype: str = "bf16"
    router_bias: str = "none"  # "none" | "normal" | "zipf"
    shared_intermediate: int = 0


CONFIGS = {
    "c1_tiny_f32": MoeShape("c1_tiny_f32", 256, 8, 2, 512, 16, 0, dtype="f32"),
    "c2_30b_a3b_decode": MoeShape("c2_30b_a3b_decode", 2048, 128, 8, 768, 64, 1),
    "c3_30b_a3b_prefill": MoeShape("c3_30b_a3b_prefill", 2048, 128, 8, 768, 4096, 2, router_bias="normal"),
    "c4_next_sparse": MoeShape("c4_next_sparse", 2048, 512, 10, 512, 2048, 3, router_bias="zipf",
                               shared_intermediate=512),
    "c5_235b_prefill": MoeShape("c5_235b_prefill", 4096, 128, 8, 1536, 8192, 4),
    "c5_235b_decode": MoeShape("c5_235b_decode", 4096, 128, 8, 1536, 32, 4),
}


def scaled(shape: MoeShape, tokens: int) -> MoeShape:
    return dataclasses.replace(shape, tokens=tokens, name=f"{shape.name}_t{tokens}")


def make_layer(shape: MoeShape, device="cuda", weights_dtype=torch.bfloat16, chunk_experts: int = 16):
    """Returns a dict of tensors: x, logits, gate_up, down, router (and shared_*)."""
    g = torch.Generator(device=device)
    g.manual_seed(shape.seed)
    H, E, I, T = shape.hidden, shape.experts, shape.intermediate, shape.tokens
    wd = torch.float32 if shape.dtype == "f32" else weights_dtype

    def normal(size, std, dtype):
        out = torch.empty(size, dtype=dtype, device=device)
        if len(size) == 3:  # generate per expert chunk to bound f32 temporaries
            for e0 in range(0, size[0], chunk_experts):
                e1 = min(size[0], e0 + chunk_experts)
                out[e0:e1] = (torch.randn((e1 - e0, *size[1:]), generator=g, device=device) * std).to(dtype)
        else:
            out.copy_((torch.randn(size, generator=g, device=device) * std).to(dtype))
        return out

    router = normal((E, H), 0.02, torch.float32)
    gate_up = normal((E, 2 * I, H), 0.02, wd)
    down = normal((E, H, I), 0.02, wd)
    x = normal((T, H), 1.0, wd)
    bias = torch.zeros(E, device=device)
    if shape.router_bias == "normal":
        bias = torch.randn(E, generator=g, device=device)
    elif shape.router_bias == "zipf":
        # Zipf(s=1.1) popularity: expert of popularity rank r gets log r^-1.1.
        order = torch.randperm(E, generator=g, device=device)
        ranks = torch.empty(E, device=device)
        ranks[order] = torch.arange(1, E + 1, device=device, dtype=torch.float32)
        bias = -1.1 * torch.log(ranks)
    logits = x.float() @ router.t() + bias
    logits = logits.to(wd) if wd != torch.float32 else logits
    out = {"x": x, "logits": logits, "gate_up": gate_up, "down": down, "router": router, "bias": bias}
    if shape.shared_intermediate:
        Is = shape.shared_intermediate
        out["shared_gate_up"] = normal((2 * Is, H), 0.02, wd)
        out["shared_down"] = normal((H, Is), 0.02, wd)
        out["shared_gate"] = normal((1, H), 0.02, wd)
    return out


def algorithmic_work(shape: MoeShape, distinct_experts: int):
    """(FLOPs, HBM bytes) of one layer pass, as counted for the roofline:
    F = 6 A H I (+ 6 T H Is + 2 T H shared); B = touched experts' BF16 weights
    once + x + logits + output (+ shared weights and gate)."""
    T, H, I, K = shape.tokens, shape.hidden, shape.intermediate, shape.top_k
    a = T * K
    flops = 6 * a * H * I
    bytes_ = distinct_experts * 3 * H * I * 2 + T * H * 2 + T * shape.experts * 2 + T * H * 2
    if shape.shared_intermediate:
        flops += 6 * T * H * shape.shared_intermediate + 2 * T * H
        bytes_ += 3 * H * shape.shared_intermediate * 2 + H * 2
    return flops, bytes_
