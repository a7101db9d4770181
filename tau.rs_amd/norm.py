"""Host mirror of the reference's centered RMSNorm and of the decoder layer's
feed-forward half around a sparse-MoE block.

* ``CenteredRmsNorm``          crates/models/src/components/rms_norm.rs:20-123
                               (``forward`` :107-123, ``add_residual_and_normalize``
                               :39-61 and its unfused form :66-74)
* ``moe_feed_forward``         crates/models/src/qwen3_5_common/decoder.rs:95-116
                               (post-attention residual + norm, the feed-forward,
                               then ``residual_sum + feed_forward(normalized)``)

Every step runs in libtau_moe_hip.so: the residual add and the norm in one
kernel, the MoE block with the final residual add fused into its last epilogue.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from . import ffi


class CenteredRmsNorm:
    """Zero-centred RMSNorm: y = x / sqrt(mean(x^2) + eps) * (1 + weight), f32
    arithmetic, rounded once to the input dtype (f32 or BF16)."""

    def __init__(self, weight: torch.Tensor, eps: float):
        if weight.dim() != 1 or weight.dtype not in (torch.float32, torch.bfloat16) or not weight.is_cuda:
            raise ValueError("the HIP norm takes a 1-D f32 or BF16 device weight")
        if not (eps > 0.0) or not math.isfinite(eps):
            raise ValueError("RMSNorm epsilon must be positive and finite")
        self.weight = weight.contiguous()
        self.eps = float(eps)

    def _check(self, x: torch.Tensor) -> None:
        if x.shape[-1] != self.weight.numel() or x.dtype != self.weight.dtype:
            raise ValueError("norm input must end in the weight's width and share its dtype")

    def forward(self, x: torch.Tensor, stream=None) -> torch.Tensor:
        self._check(x)
        return ffi.centered_rms_norm(x.contiguous(), self.weight, self.eps, stream=stream)

    __call__ = forward

    def add_residual_and_normalize(self, residual: torch.Tensor, branch: torch.Tensor,
                                   stream=None) -> Tuple[torch.Tensor, torch.Tensor]:
        """(residual + branch rounded to the dtype, its normalization), one kernel."""
        self._check(residual)
        if branch.shape != residual.shape or branch.dtype != residual.dtype:
            raise ValueError("residual and branch must share shape and dtype")
        return ffi.fused_residual_rms_norm(residual.contiguous(), branch.contiguous(), self.weight, self.eps,
                                           stream=stream)


def moe_feed_forward(xs: torch.Tensor, branch: torch.Tensor, post_norm: CenteredRmsNorm, block,
                     logits: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """The decoder layer after its token mixer: residual_sum = xs + branch,
    normalized = post_norm(residual_sum), output = residual_sum + block(normalized),
    with the final add fused into the block's last epilogue.  xs, branch: BF16
    [T, H]; block: a SparseMoeBlock; logits: optional precomputed router logits
    for `normalized` (computed by the block's router otherwise)."""
    residual_sum, normalized = post_norm.add_residual_and_normalize(xs, branch, stream=stream)
    return block.forward(normalized, logits=logits, stream=stream, residual=residual_sum)
