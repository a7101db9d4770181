"""ctypes binding of libtau_moe_hip.so (declared in include/tau_moe.h).

Torch is used only as device-memory and stream plumbing: every call passes raw
device pointers and the current HIP stream to the C ABI.  The library must be
built (``build.py``); loading fails loudly when it is missing, and there is no
CPU or PyTorch fallback for any operation.
"""
from __future__ import annotations

import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
# TAU_MOE_LIBRARY overrides the library file (e.g. an alternative build).
LIB_PATH = os.environ.get("TAU_MOE_LIBRARY") or os.path.join(HERE, "libtau_moe_hip.so")

# Every symbol declared in include/tau_moe.h.
EXPORTS = (
    "tau_launch_moe_routing_fp32",
    "tau_launch_moe_prefill_dispatch",
    "tau_launch_moe_prefill_combine",
    "tau_launch_moe_prefill_gemm",
    "tau_launch_moe_prefill",
    "tau_launch_silu_and_mul",
    "tau_launch_moe_shared_combine",
    "tau_launch_linear_bf16_fp32",
    "tau_launch_moe_decode_gemm",
    "tau_launch_fused_bf16_moe_decode",
    "tau_moe_prefill_capacity",
    "tau_moe_select_tile_rows",
    "tau_moe_workspace_bytes",
    "tau_launch_moe_routing_ex",
    "tau_launch_moe_prefill_dispatch_ex",
    "tau_launch_moe_prefill_combine_ex",
    "tau_launch_moe_prefill_ex",
    "tau_launch_moe_shared_expert_ex",
    "tau_launch_moe_grouped_gemm_ex",
    "tau_launch_moe_decode_projection_ex",
    "tau_moe_pack_weights",
    "tau_launch_moe_router_ex",
    "tau_launch_moe_router_route_ex",
    "tau_launch_moe_routing_shared_ex",
    "tau_launch_moe_router_route_shared_ex",
    "tau_launch_fused_residual_rms_norm",
    "tau_launch_centered_rms_norm_configured",
    "tau_launch_centered_rms_norm",
    "tau_moe_build_target",
)

# Expert weight layouts (TAU_MOE_WEIGHTS_* in include/tau_moe.h).
WEIGHTS_ROW_MAJOR = 0
WEIGHTS_FRAG16 = 1


class TauGemmTile(ctypes.Structure):
    _fields_ = [("m", ctypes.c_int), ("n", ctypes.c_int), ("k", ctypes.c_int),
                ("warps", ctypes.c_int), ("stages", ctypes.c_int)]


class TauDecodeProfile(ctypes.Structure):
    _fields_ = [("backend", ctypes.c_int), ("n", ctypes.c_int), ("k", ctypes.c_int),
                ("warps", ctypes.c_int), ("stages", ctypes.c_int)]


class LaunchError(RuntimeError):
    """Nonzero launch status (mirrors the reference's LaunchError{code,kernel})."""

    def __init__(self, code: int, kernel: str):
        super().__init__(f"{kernel} launch failed with status {code}")
        self.code = code
        self.kernel = kernel


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() (no fallback exists)")
    L = ctypes.CDLL(LIB_PATH)
    p, i, i64, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
    sig = {
        "tau_launch_moe_routing_fp32": [p, p, i, p],
        "tau_launch_moe_prefill_dispatch": [p, p, p, p, p, i, i, i, p],
        "tau_launch_moe_prefill_combine": [p, p, p, i, i, p],
        "tau_launch_moe_prefill_gemm": [p, p, p, p, p, p, i, i, i, i, i, p, p, p],
        "tau_launch_moe_prefill": [p] * 13 + [i] * 4 + [p, p, p, p],
        "tau_launch_silu_and_mul": [p, p, i, i, i, p],
        "tau_launch_moe_shared_combine": [p, p, p, p, p, i, i, p],
        "tau_launch_linear_bf16_fp32": [p, p, p, i, i, i, p],
        "tau_launch_moe_decode_gemm": [p, p, p, i, i, i, p, p, p],
        "tau_launch_fused_bf16_moe_decode": [p] * 13 + [i] * 4 + [p, p, p, p],
        "tau_moe_prefill_capacity": [i, i, i, i],
        "tau_moe_select_tile_rows": [i, i, i, i, i],
        "tau_moe_workspace_bytes": [i, i, i, i, i, i, p],
        "tau_launch_moe_routing_ex": [p, i, p, i, i, i, p],
        "tau_launch_moe_prefill_dispatch_ex": [p, i, p, p, p, p, p, i, i, i, i, i, p],
        "tau_launch_moe_prefill_combine_ex": [p, p, p, i, i, i, i, p, p],
        "tau_launch_moe_prefill_ex": [p, p, i, p, p, p, p, p, p, p, p, p, p, i, i, i, i, i, i, i, i, p, p, p],
        "tau_launch_moe_shared_expert_ex": [p] * 8 + [i, i, i, i, p, p],
        "tau_launch_moe_grouped_gemm_ex": [p] * 7 + [i] * 9 + [p, p],
        "tau_launch_moe_decode_projection_ex": [p] * 8 + [i] * 8 + [p, p],
        "tau_moe_pack_weights": [p, p, i, i, i, p],
        "tau_launch_moe_router_ex": [p, p, p, p, i, i, i, p],
        "tau_launch_moe_router_route_ex": [p, p, p, p, p, i, i, i, i, p],
        "tau_launch_moe_routing_shared_ex": [p, i, p, i, i, i, p],
        "tau_launch_moe_router_route_shared_ex": [p, p, p, p, p, i, i, i, i, p],
        "tau_launch_fused_residual_rms_norm": [p, p, p, p, p, i, i, f32, i, p, i],
        "tau_launch_centered_rms_norm_configured": [p, p, p, i, i, f32, i, p, i],
        "tau_launch_centered_rms_norm": [p, p, p, i, i, f32, i, p],
    }
    for name, args in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = i
    L.tau_moe_prefill_capacity.restype = i64
    L.tau_moe_build_target.argtypes = []
    L.tau_moe_build_target.restype = ctypes.c_char_p
    _lib = L
    return L


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def stream_ptr(stream=None):
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def check(code: int, kernel: str) -> None:
    if code != 0:
        raise LaunchError(code, kernel)


ROUTE_RAW_WEIGHTS = 0x100  # TAU_MOE_ROUTE_RAW_WEIGHTS: keep the selected probabilities unnormalised


def _dtype_code(t: torch.Tensor, raw_weights: bool = False) -> int:
    flag = ROUTE_RAW_WEIGHTS if raw_weights else 0
    if t.dtype == torch.float32:
        return 0 | flag
    if t.dtype == torch.bfloat16:
        return 1 | flag
    raise TypeError(f"unsupported dtype {t.dtype}")


def capacity(tokens: int, experts: int, top_k: int, tile_rows: int) -> int:
    return int(lib().tau_moe_prefill_capacity(tokens, experts, top_k, tile_rows))


def select_tile_rows(tokens, experts, top_k, hidden, intermediate) -> int:
    return int(lib().tau_moe_select_tile_rows(tokens, experts, top_k, hidden, intermediate))


def workspace_bytes(tokens, hidden, intermediate, experts, top_k, tile_rows):
    out = (ctypes.c_size_t * 7)()
    check(lib().tau_moe_workspace_bytes(tokens, hidden, intermediate, experts, top_k, tile_rows, out),
          "workspace query")
    return list(out)


def routing_ex(logits, routes, experts, top_k, stream=None, raw_weights=False):
    t = logits.shape[0]
    check(lib().tau_launch_moe_routing_ex(ptr(logits), _dtype_code(logits, raw_weights), ptr(routes), t, experts,
                                          top_k,
                                          stream_ptr(stream)), "MoE routing")


def dispatch_ex(logits, routes, meta, offsets, slots, tiles, tokens, experts, top_k, tile_rows, cap,
                stream=None, raw_weights=False):
    code = lib().tau_launch_moe_prefill_dispatch_ex(
        ptr(logits), _dtype_code(logits, raw_weights) if logits is not None else 0, ptr(routes), ptr(meta), ptr(offsets),
        ptr(slots), ptr(tiles), tokens, experts, top_k, tile_rows, cap, stream_ptr(stream))
    check(code, "MoE dispatch")


def prefill_ex(x, logits, gate_up, down, ws, output, experts, top_k, tile_rows, receipts=None, stream=None,
               weight_layout=WEIGHTS_ROW_MAJOR, residual=None, raw_weights=False):
    t, h = x.shape
    i = down.shape[2]
    code = lib().tau_launch_moe_prefill_ex(
        ptr(x), ptr(logits), _dtype_code(logits, raw_weights) if logits is not None else 0, ptr(gate_up), ptr(down),
        ptr(ws["routes"]), ptr(ws["meta"]),
        ptr(ws["offsets"]), ptr(ws["slots"]), ptr(ws["tiles"]), ptr(ws["activated"]),
        ptr(ws["contributions"]), ptr(output), t, h, i, experts, top_k, tile_rows, ws["capacity"],
        weight_layout, ptr(residual), ptr(receipts), stream_ptr(stream))
    check(code, "MoE grouped prefill")


def shared_expert_ex(x, gate_up_s, down_s, gate_weight, routed, activated_ws, shared_ws, output, stream=None,
                     weight_layout=WEIGHTS_ROW_MAJOR, residual=None):
    t, h = x.shape
    i_s = down_s.shape[1]
    code = lib().tau_launch_moe_shared_expert_ex(
        ptr(x), ptr(gate_up_s), ptr(down_s), ptr(gate_weight), ptr(routed), ptr(activated_ws), ptr(shared_ws),
        ptr(output), t, h, i_s, weight_layout, ptr(residual), stream_ptr(stream))
    check(code, "MoE shared expert")


def grouped_gemm_ex(a, w, ws, out, tokens, hidden, intermediate, experts, top_k, tile_rows, projection,
                    receipt=None, stream=None, weight_layout=WEIGHTS_ROW_MAJOR):
    code = lib().tau_launch_moe_grouped_gemm_ex(
        ptr(a), ptr(w), ptr(ws["routes"]), ptr(ws["slots"]), ptr(ws["tiles"]), ptr(ws["meta"]), ptr(out), tokens,
        hidden, intermediate, experts, top_k, tile_rows, ws["capacity"], projection, weight_layout, ptr(receipt),
        stream_ptr(stream))
    check(code, "MoE grouped GEMM")


def decode_projection_ex(a, w, ws, out, tokens, hidden, intermediate, experts, top_k, projection, receipt=None,
                         stream=None, weight_layout=WEIGHTS_ROW_MAJOR):
    """One fused-decode projection over the workspace's routes (tile_rows 16)."""
    code = lib().tau_launch_moe_decode_projection_ex(
        ptr(a), ptr(w), ptr(ws["routes"]), ptr(ws["meta"]), ptr(ws["offsets"]), ptr(ws["slots"]), ptr(ws["tiles"]),
        ptr(out), tokens, hidden, intermediate, experts, top_k, ws["capacity"], projection, weight_layout,
        ptr(receipt), stream_ptr(stream))
    check(code, "MoE decode projection")


def combine_ex(contributions, output, meta, tokens, hidden, experts, top_k, stream=None, residual=None):
    code = lib().tau_launch_moe_prefill_combine_ex(ptr(contributions), ptr(output), ptr(meta), tokens, hidden,
                                                   experts, top_k, ptr(residual), stream_ptr(stream))
    check(code, "MoE combine")


def pack_weights(w: torch.Tensor, stream=None) -> torch.Tensor:
    """FRAG16 copy of row-major BF16 weights [E, n, k] (or [n, k]); same shape,
    fragment-ordered contents (TAU_MOE_WEIGHTS_FRAG16)."""
    if w.dtype != torch.bfloat16 or not w.is_contiguous():
        raise TypeError("pack_weights expects contiguous BF16 weights")
    e, n, k = (1, *w.shape) if w.dim() == 2 else w.shape
    out = torch.empty_like(w)
    check(lib().tau_moe_pack_weights(ptr(w), ptr(out), e, n, k, stream_ptr(stream)), "MoE weight pack")
    return out


def router_route_ex(x: torch.Tensor, weight: torch.Tensor, bias, logits: torch.Tensor, routes: torch.Tensor,
                    top_k: int, stream=None, raw_weights=False):
    """logits f32 [T, E] and routes [T, 2K] from x BF16 [T, H] in one call
    (two calls, projection then routing, for unnormalised weights)."""
    t, h = x.shape
    e = weight.shape[0]
    if raw_weights:
        router_ex(x, weight, bias, logits, stream=stream)
        routing_ex(logits, routes, e, top_k, stream=stream, raw_weights=True)
        return
    check(lib().tau_launch_moe_router_route_ex(ptr(x), ptr(weight), ptr(bias), ptr(logits), ptr(routes), t, h, e,
                                               top_k, stream_ptr(stream)), "MoE router + routing")


def routing_shared_ex(logits, routes, experts, top_k, stream=None, raw_weights=False):
    """routes [T, 2(K+1)] from logits [T, E+1]: routed top-K, then (E, sigmoid(gate))."""
    t = logits.shape[0]
    check(lib().tau_launch_moe_routing_shared_ex(ptr(logits), _dtype_code(logits, raw_weights), ptr(routes), t,
                                                 experts, top_k,
                                                 stream_ptr(stream)), "MoE routing with shared expert")


def router_route_shared_ex(x, weight, bias, logits, routes, experts, top_k, stream=None, raw_weights=False):
    """logits f32 [T, E+1] and routes [T, 2(K+1)] from x BF16 [T, H]; weight [E+1, H]."""
    t, h = x.shape
    if raw_weights:
        router_ex(x, weight, bias, logits, stream=stream)
        routing_shared_ex(logits, routes, experts, top_k, stream=stream, raw_weights=True)
        return
    check(lib().tau_launch_moe_router_route_shared_ex(ptr(x), ptr(weight), ptr(bias), ptr(logits), ptr(routes), t, h,
                                                      experts, top_k, stream_ptr(stream)),
          "MoE router + routing with shared expert")


def router_ex(x: torch.Tensor, weight: torch.Tensor, bias, logits: torch.Tensor, stream=None):
    """logits f32 [T, E] = x BF16 [T, H] . weight BF16 [E, H]^T (+ bias f32 [E])."""
    t, h = x.shape
    e = weight.shape[0]
    check(lib().tau_launch_moe_router_ex(ptr(x), ptr(weight), ptr(bias), ptr(logits), t, h, e, stream_ptr(stream)),
          "MoE router")


def _norm_operands(x: torch.Tensor, weight: torch.Tensor):
    if (x.dim() < 1 or weight.dim() != 1 or x.shape[-1] != weight.numel() or x.dtype != weight.dtype
            or not x.is_contiguous() or not weight.is_contiguous()):
        raise ValueError("norm input must be contiguous [..., columns] with a contiguous [columns] weight of its dtype")
    columns = x.shape[-1]
    return x.numel() // columns, columns, _dtype_code(x)


def centered_rms_norm(x: torch.Tensor, weight: torch.Tensor, epsilon: float, out=None, preferred_bytes: int = 16,
                      stream=None) -> torch.Tensor:
    """(x / sqrt(mean(x^2) + eps)) * (1 + weight) over the last dimension, f32
    arithmetic, rounded once to x's dtype (f32 or BF16)."""
    rows, columns, dt = _norm_operands(x, weight)
    out = torch.empty_like(x) if out is None else out
    check(lib().tau_launch_centered_rms_norm_configured(ptr(x), ptr(weight), ptr(out), rows, columns,
                                                        float(epsilon), dt, stream_ptr(stream), preferred_bytes),
          "centered RMSNorm")
    return out


def fused_residual_rms_norm(x: torch.Tensor, branch: torch.Tensor, weight: torch.Tensor, epsilon: float,
                            preferred_bytes: int = 16, stream=None):
    """(residual, normalized): residual = x + branch rounded to the dtype, then
    the centered RMSNorm of the residual; one pass over the rows."""
    rows, columns, dt = _norm_operands(x, weight)
    if branch.shape != x.shape or branch.dtype != x.dtype or not branch.is_contiguous():
        raise ValueError("branch must be contiguous and shaped like the input")
    residual = torch.empty_like(x)
    out = torch.empty_like(x)
    check(lib().tau_launch_fused_residual_rms_norm(ptr(x), ptr(branch), ptr(weight), ptr(residual),
                                                   ptr(out), rows, columns, float(epsilon), dt, stream_ptr(stream),
                                                   preferred_bytes),
          "fused residual RMSNorm")
    return residual, out
