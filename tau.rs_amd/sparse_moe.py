"""Host-side mirror of the reference's sparse-MoE operator interface.

Names, argument meaning and error behaviour follow the reference's Rust owners
(paths relative to the tau.rs root):

* ``SparseMoeConfig.validate``  crates/models/src/components/sparse_moe/config.rs:52-78
* ``MoePrefillTile``            crates/cuda-kernels/src/moe/config.rs:12-158 (parse,
                                validate, ``values``, ``rows``)
* ``moe_prefill_capacity``      crates/cuda-kernels/src/moe/prefill.rs:11-30
* ``MoePrefillRunner``          crates/models/src/components/cuda/fused_moe/prefill.rs:
                                workspace grown to the next power of two >= T
                                (:330-340), ``calls()`` counter (:212-216),
                                ``workspace_info`` and ``executed_tiles`` receipts
* ``SparseMoeBlock.forward``    crates/models/src/components/sparse_moe.rs:102-151
                                (routed experts, then the shared-expert combine)

Every compute step runs in libtau_moe_hip.so; this module only validates,
owns device workspaces (torch tensors as plumbing) and sequences launches.
"""
from __future__ import annotations

import dataclasses
from typing import Optional

import torch

from . import ffi


@dataclasses.dataclass
class SharedExpertConfig:
    intermediate_size: int
    gated: bool = True  # sigmoid(x . w_s) gate without bias


@dataclasses.dataclass
class SparseMoeConfig:
    hidden_size: int
    expert_intermediate_size: int
    num_experts: int
    experts_per_token: int
    normalize_selected_weights: bool = True
    shared_expert: Optional[SharedExpertConfig] = None

    def validate(self) -> None:
        """Raises ValueError with the reference's messages (config.rs:52-78)."""
        if (self.hidden_size == 0 or self.expert_intermediate_size == 0 or self.num_experts == 0
                or self.experts_per_token == 0):
            raise ValueError("sparse MoE dimensions and expert counts must be non-zero")
        if self.experts_per_token > self.num_experts:
            raise ValueError("sparse MoE experts_per_token cannot exceed num_experts")
        if self.shared_expert is not None and self.shared_expert.intermediate_size == 0:
            raise ValueError("sparse MoE shared-expert intermediate size must be non-zero")
        if self.num_experts > 512 or self.experts_per_token > 32:
            raise ValueError("the HIP path supports num_experts <= 512 and experts_per_token <= 32")


@dataclasses.dataclass(frozen=True)
class MoePrefillTile:
    """Five tile words M,N,K,warps,stages (config.rs:12-20).  M selects the CDNA4
    row block (16/32 = weight-streaming kernels, 64/128/256 = LDS-tiled MFMA); the
    remaining words are validated against the reference catalog."""
    m: int = 16
    n: int = 16
    k: int = 16
    warps: int = 1
    stages: int = 1

    def __post_init__(self):
        ok = (self.m in (16, 32, 64, 128, 256) and self.n in (16, 32, 64, 128) and self.k in (16, 32, 64, 128)
              and self.warps in (1, 2, 4, 8) and self.stages in (1, 2))
        if not ok:
            raise ValueError(f"unsupported MoE prefill tile {self.values()}; expected M=16|32|64|128|256, "
                             "N=16|32|64|128, K=16|32|64|128, warps=1|2|4|8, stages=1|2")

    @classmethod
    def parse(cls, text: str) -> "MoePrefillTile":
        try:
            vals = [int(v) for v in text.split(",")]
        except ValueError:
            raise ValueError("expected MoE prefill M,N,K,warps,stages") from None
        if len(vals) != 5:
            raise ValueError("expected five MoE prefill values: M,N,K,warps,stages")
        return cls(*vals)

    def values(self):
        return [self.m, self.n, self.k, self.warps, self.stages]

    def rows(self) -> int:
        return self.m

    def __str__(self):
        return ",".join(str(v) for v in self.values())


def moe_prefill_capacity(tokens: int, experts: int = 256, top_k: int = 8, tile_rows: int = 16) -> Optional[int]:
    """None for invalid token counts, like the reference's Option (prefill.rs:17-30)."""
    if tokens <= 0 or tokens > (1 << 20):
        return None
    c = ffi.capacity(tokens, experts, top_k, tile_rows)
    return None if c < 0 else c


def _next_pow2(n: int) -> int:
    p = 1
    while p < n:
        p <<= 1
    return p


class MoePrefillRunner:
    """Owns the routed-expert weights and the grouped-prefill workspaces.

    weight_layout: "auto" keeps a FRAG16 copy of the weights (1 KB MFMA operand
    fragments, see include/tau_moe.h) when the shape allows it (hidden and
    intermediate multiples of 64) and the caller's row-major tensors otherwise;
    "row_major" / "frag16" force one layout."""

    def __init__(self, config: SparseMoeConfig, gate_up: torch.Tensor, down: torch.Tensor,
                 tile_rows: Optional[int] = None, weight_layout: str = "auto", fold_shared: bool = False):
        """fold_shared: the banks hold one more expert, the shared expert, which
        every token takes at rank K (routes from tau_launch_moe_routing_shared_ex);
        the runner then launches E+1 experts and K+1 picks."""
        config.validate()
        if fold_shared:
            config = dataclasses.replace(config, num_experts=config.num_experts + 1,
                                         experts_per_token=config.experts_per_token + 1, shared_expert=None)
        E, I, H = config.num_experts, config.expert_intermediate_size, config.hidden_size
        if gate_up.shape != (E, 2 * I, H) or down.shape != (E, H, I):
            raise ValueError("packed expert weights must be gate_up [E,2I,H] and down [E,H,I]")
        if gate_up.dtype != torch.bfloat16 or down.dtype != torch.bfloat16 or not gate_up.is_cuda:
            raise ValueError("the HIP path takes contiguous BF16 device weights")
        self.config = config
        self.raw_weights = not config.normalize_selected_weights
        packable = H % 64 == 0 and I % 64 == 0
        if weight_layout not in ("auto", "row_major", "frag16"):
            raise ValueError(f"unknown weight layout {weight_layout!r}")
        if weight_layout == "frag16" and not packable:
            raise ValueError("frag16 weights need hidden and intermediate sizes divisible by 64")
        if weight_layout == "frag16" or (weight_layout == "auto" and packable):
            self.layout = ffi.WEIGHTS_FRAG16
            self.gate_up = ffi.pack_weights(gate_up.contiguous())
            self.down = ffi.pack_weights(down.contiguous())
        else:
            self.layout = ffi.WEIGHTS_ROW_MAJOR
            self.gate_up = gate_up.contiguous()
            self.down = down.contiguous()
        self.fixed_tile_rows = tile_rows
        self._ws = None
        self._ws_key = None
        self._calls = 0
        self._receipts = torch.zeros(10, dtype=torch.int32, device=gate_up.device)

    def calls(self) -> int:
        return self._calls

    def tile_rows_for(self, tokens: int) -> int:
        c = self.config
        if self.fixed_tile_rows:
            return self.fixed_tile_rows
        return ffi.select_tile_rows(tokens, c.num_experts, c.experts_per_token, c.hidden_size,
                                    c.expert_intermediate_size)

    def workspace(self, tokens: int, tile_rows: int):
        """Workspaces sized for the next power of two >= tokens; reused while they fit."""
        c = self.config
        alloc_tokens = _next_pow2(tokens)
        key = (tile_rows,)
        if self._ws is not None and self._ws_key == key and self._ws["tokens"] >= tokens:
            return self._ws
        sizes = ffi.workspace_bytes(alloc_tokens, c.hidden_size, c.expert_intermediate_size, c.num_experts,
                                    c.experts_per_token, tile_rows)
        dev = self.gate_up.device
        cap = ffi.capacity(alloc_tokens, c.num_experts, c.experts_per_token, tile_rows)
        ws = {
            "tokens": alloc_tokens,
            "capacity": cap,
            "routes": torch.empty(sizes[0] // 4, dtype=torch.float32, device=dev),
            "meta": torch.empty(sizes[1] // 4, dtype=torch.int32, device=dev),
            "offsets": torch.empty(sizes[2] // 4, dtype=torch.int32, device=dev),
            "slots": torch.empty(sizes[3] // 4, dtype=torch.int32, device=dev),
            "tiles": torch.empty(sizes[4] // 4, dtype=torch.int32, device=dev),
            "activated": torch.empty(sizes[5] // 2, dtype=torch.bfloat16, device=dev),
            "contributions": torch.empty(sizes[6] // 2, dtype=torch.bfloat16, device=dev),
        }
        self._ws, self._ws_key = ws, key
        return ws

    def workspace_info(self):
        if self._ws is None:
            return None
        return (self._ws["tokens"], self._ws["capacity"], self._ws["slots"].data_ptr())

    def executed_tiles(self):
        return self._receipts.view(2, 5).tolist()

    def forward(self, x: torch.Tensor, logits: Optional[torch.Tensor], out: Optional[torch.Tensor] = None,
                stream=None, residual: Optional[torch.Tensor] = None, router=None) -> torch.Tensor:
        """Routed-expert output; with `residual` (BF16 [T, H]) returns
        bf16(output + residual), the layer's residual add fused in the combine.
        logits None: `router(routes)` writes the [T, 2K] routes into the
        workspace's routes buffer (the router projection with the routing,
        tau_launch_moe_router_route_ex, or the shared-expert routing) and the
        layer starts from them."""
        c = self.config
        if x.dim() != 2 or x.shape[1] != c.hidden_size or x.dtype != torch.bfloat16:
            raise ValueError("input must be BF16 [tokens, hidden]")
        if logits is None and router is None:
            raise ValueError("pass router logits or a routes producer")
        if logits is not None and logits.shape != (x.shape[0], c.num_experts):
            raise ValueError("router logits must be [tokens, num_experts]")
        tokens = x.shape[0]
        tile_rows = self.tile_rows_for(tokens)
        ws = self.workspace(tokens, tile_rows)
        # Capacity of the allocation covers any token count up to ws["tokens"].
        if out is None:
            out = torch.empty_like(x)
        x = x.contiguous()
        if logits is None:
            router(ws["routes"])
        else:
            logits = logits.contiguous()
        ffi.prefill_ex(x, logits, self.gate_up, self.down, ws, out, c.num_experts,
                       c.experts_per_token, tile_rows, receipts=self._receipts, stream=stream,
                       weight_layout=self.layout, residual=residual, raw_weights=self.raw_weights)
        self._calls += 1
        return out

    def plan_views(self, tokens: int):
        """Device views of the last dispatch (routes [T,2K], meta, offsets, slots, tiles)."""
        ws = self._ws
        c = self.config
        K, E = c.experts_per_token, c.num_experts
        return {
            "routes": ws["routes"][: tokens * 2 * K].view(tokens, 2 * K),
            "meta": ws["meta"][: 2 * E + 2],
            "offsets": ws["offsets"][: E + 1],
            "slots": ws["slots"],
            "tiles": ws["tiles"],
        }


class SparseMoeBlock:
    """Routed experts plus the optional always-on shared expert (sparse_moe.rs:102-251).

    With `router_weight` (BF16 [E, H]) and optional `router_bias` (f32 [E]) the
    block computes its own router logits in f32 (routing.rs:91-93) when
    `forward` is called without them."""

    def __init__(self, config: SparseMoeConfig, gate_up, down, shared_gate_up=None, shared_down=None,
                 shared_gate=None, tile_rows: Optional[int] = None, weight_layout: str = "auto",
                 router_weight: Optional[torch.Tensor] = None, router_bias: Optional[torch.Tensor] = None,
                 fold_shared: Optional[bool] = None):
        config.validate()
        E, H, I, K = config.num_experts, config.hidden_size, config.expert_intermediate_size, config.experts_per_token
        se = config.shared_expert
        if se is not None:
            if shared_gate_up is None or shared_down is None:
                raise ValueError("shared expert weights missing")
            if se.gated and shared_gate is None:
                raise ValueError("shared expert gate weight missing")
        # A gated shared expert with the experts' intermediate size runs as
        # expert E of the routed schedule (default when possible).
        foldable = (se is not None and se.gated and se.intermediate_size == I and K + 1 <= 32
                    and tuple(shared_gate_up.shape) == (2 * I, H) and tuple(shared_down.shape) == (H, I))
        self.folded = foldable if fold_shared is None else bool(fold_shared)
        if self.folded and not foldable:
            raise ValueError("folding needs a gated shared expert with the experts' intermediate size and K < 32")
        if self.folded:
            gu_all = torch.cat([gate_up, shared_gate_up.unsqueeze(0).to(gate_up.dtype)], 0)
            dn_all = torch.cat([down, shared_down.unsqueeze(0).to(down.dtype)], 0)
            self.runner = MoePrefillRunner(config, gu_all, dn_all, tile_rows, weight_layout, fold_shared=True)
            del gu_all, dn_all
        else:
            self.runner = MoePrefillRunner(config, gate_up, down, tile_rows, weight_layout)
        self.config = config
        self.router = None
        if router_weight is not None:
            if router_weight.shape != (E, H) or router_weight.dtype != torch.bfloat16:
                raise ValueError("router weight must be BF16 [num_experts, hidden]")
            if router_bias is not None and (router_bias.shape != (E,) or router_bias.dtype != torch.float32):
                raise ValueError("router bias must be f32 [num_experts]")
            w, b = router_weight.contiguous(), None if router_bias is None else router_bias.contiguous()
            if self.folded:  # the shared gate row w_s after the router rows, no bias for it
                w = torch.cat([w, shared_gate.reshape(1, H).to(torch.bfloat16)], 0).contiguous()
                if b is not None:
                    b = torch.cat([b, torch.zeros(1, dtype=b.dtype, device=b.device)]).contiguous()
            self.router = (w, b)
        self._logits = None
        self._gate_logits = None
        self.shared = None
        if self.folded:
            self.shared_gate = shared_gate.reshape(1, H).to(torch.bfloat16).contiguous()
        elif se is not None:
            gu, dn = shared_gate_up.contiguous(), shared_down.contiguous()
            Is, H = config.shared_expert.intermediate_size, config.hidden_size
            self.shared_layout = ffi.WEIGHTS_ROW_MAJOR
            if self.runner.layout == ffi.WEIGHTS_FRAG16 and Is % 64 == 0 and H % 64 == 0:
                gu, dn = ffi.pack_weights(gu), ffi.pack_weights(dn)
                self.shared_layout = ffi.WEIGHTS_FRAG16
            self.shared = (gu, dn, shared_gate.contiguous() if config.shared_expert.gated else None)
        self._shared_ws = None

    def logits(self, x: torch.Tensor, stream=None) -> torch.Tensor:
        """Router scores f32 [T, E] (x . W_r^T + b); with the shared expert
        folded in, [T, E+1] with the gate logit x . w_s last."""
        if self.router is None:
            raise ValueError("block built without router weights: pass logits to forward")
        out = self._logits_buffer(x.shape[0], x.device)
        ffi.router_ex(x, self.router[0], self.router[1], out, stream=stream)
        return out

    def _logits_buffer(self, T: int, device):
        E = self.config.num_experts + (1 if self.folded else 0)
        if self._logits is None or self._logits.shape[0] < T:
            self._logits = torch.empty(_next_pow2(T), E, dtype=torch.float32, device=device)
        return self._logits[:T]

    def _fused_router(self, x: torch.Tensor, stream=None):
        """routes(routes_buffer) for the router + routing call (with the shared
        expert's gate when folded), or None without router weights."""
        if self.router is None:
            return None
        w, b = self.router
        logits = self._logits_buffer(x.shape[0], x.device)
        E, K = self.config.num_experts, self.config.experts_per_token
        raw = not self.config.normalize_selected_weights
        if self.folded:
            return lambda routes: ffi.router_route_shared_ex(x, w, b, logits, routes, E, K, stream=stream,
                                                             raw_weights=raw)
        return lambda routes: ffi.router_route_ex(x, w, b, logits, routes, K, stream=stream, raw_weights=raw)

    def _shared_routes(self, x: torch.Tensor, logits: torch.Tensor, stream=None):
        """routes(routes_buffer) from caller logits for the folded shared expert:
        [T, E+1] as given, or [T, E] plus the gate column x . w_s projected here."""
        E, K = self.config.num_experts, self.config.experts_per_token
        T = x.shape[0]
        if logits.shape == (T, E + 1):
            ext = logits.contiguous()
        elif logits.shape == (T, E):
            if self._gate_logits is None or self._gate_logits.shape[0] < T:
                self._gate_logits = torch.empty(_next_pow2(T), 1, dtype=torch.float32, device=x.device)
            gate = self._gate_logits[:T]
            ffi.router_ex(x, self.shared_gate, None, gate, stream=stream)
            ext = torch.cat([logits.float(), gate], 1) if logits.dtype != torch.float32 else torch.cat([logits, gate], 1)
        else:
            raise ValueError("router logits must be [tokens, num_experts] (or + 1 shared gate column)")
        raw = not self.config.normalize_selected_weights
        return lambda routes: ffi.routing_shared_ex(ext, routes, E, K, stream=stream, raw_weights=raw)

    def forward(self, x: torch.Tensor, logits: Optional[torch.Tensor] = None, stream=None,
                residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Block output; with `residual` (BF16 [T, H]) the layer's residual add
        (decoder.rs:96-116) is fused into the block's last epilogue.  Without
        logits the router runs on x together with the routing
        (tau_launch_moe_router_route_ex; the projection is kept in the block's
        logits buffer) and the layer starts from those routes."""
        router = None
        x = x.contiguous()
        if logits is None:
            router = self._fused_router(x, stream=stream)
            if router is None:
                raise ValueError("block built without router weights: pass logits to forward")
        elif self.folded:
            router, logits = self._shared_routes(x, logits, stream=stream), None
        if residual is not None and (residual.shape != x.shape or residual.dtype != torch.bfloat16):
            raise ValueError("residual must be BF16 shaped like the input")
        if self.shared is None:  # no shared expert, or folded into the routed schedule
            return self.runner.forward(x, logits, stream=stream, residual=residual, router=router)
        routed = self.runner.forward(x, logits, stream=stream, router=router)
        gu, dn, gw = self.shared
        T = x.shape[0]
        Is = self.config.shared_expert.intermediate_size
        if self._shared_ws is None or self._shared_ws[0].shape[0] < T:
            n = _next_pow2(T)
            self._shared_ws = (torch.empty(n, Is, dtype=torch.bfloat16, device=x.device),
                               torch.empty(n, x.shape[1], dtype=torch.bfloat16, device=x.device))
        act, sh = self._shared_ws
        ffi.shared_expert_ex(x, gu, dn, gw, routed, act[:T], sh[:T], routed, stream=stream,
                             weight_layout=self.shared_layout, residual=residual)
        return routed

    def capture(self, x: torch.Tensor, logits: Optional[torch.Tensor] = None,
                residual: Optional[torch.Tensor] = None):
        """Records forward(x, logits, residual) into a HIP graph (the reference
        captures its prepared decode program, components/cuda/graph.rs:22-150).

        x / logits / residual are the graph's static input buffers: copy new
        values into them and call graph.replay(); the result lands in the
        returned output tensor.  One eager call first sizes the workspaces, so
        the capture allocates nothing; the library issues kernels only (no
        memset nodes).  Returns (graph, output)."""
        self.forward(x, logits, residual=residual)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = self.forward(x, logits, residual=residual)
        return graph, out
