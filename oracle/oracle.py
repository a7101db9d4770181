"""TEST INFRASTRUCTURE ONLY: ctypes front-end of the CPU parity oracle.

Loads ``oracle/libmoe_oracle.so`` (built from ``moe_oracle.c`` by the
Makefile next to this file).  Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s cpu_baseline leg may import this module, as the checker
or as the timed CPU baseline; the product path never does.

Every function here forwards to the C restatement documented in
``moe_oracle.c`` (reference citations live there, function by function):

* ``route``            routing.rs:125-257 (softmax, top-k, rank-order renorm)
* ``select_experts``   routing.rs:239-257
* ``plan``             routing.rs:215-227 (stable expert-major grouping)
* ``dispatch``         moe_dispatch.cu:11-85 layout with the stable order
* ``moe``              experts.rs:97-152 + mlp.rs:50-83 (f32 or BF16 contract)
* ``dense_mlp``        mlp.rs forward (shared expert MLP)
* ``shared_combine_*`` shared_expert.rs:68,142-159 / moe_shared.cu:17-36
* ``silu_and_mul``     silu_and_mul.cu:51-76
* ``centered_rms_norm`` rms_norm.rs:66-74,107-150,204-210 (optional residual add)
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libmoe_oracle.so")
_lib = None

ACT_SILU = 0
ACT_RELU = 1


def build() -> str:
    """Compile the oracle with its Makefile (used by build() and tests)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        f = ctypes.c_void_p
        i = ctypes.c_int
        i64 = ctypes.c_int64
        _lib.oracle_route.argtypes = [f, i, i, i, i, f, f, f]
        _lib.oracle_route.restype = i
        _lib.oracle_select_experts.argtypes = [f, i, i, f]
        _lib.oracle_select_experts.restype = i
        _lib.oracle_plan.argtypes = [f, i, i, i, f, f, f]
        _lib.oracle_plan.restype = None
        _lib.oracle_capacity.argtypes = [i64, i64, i64, i64]
        _lib.oracle_capacity.restype = i64
        _lib.oracle_dispatch.argtypes = [f, i, i, i, i, i64, f, f, f, f]
        _lib.oracle_dispatch.restype = i
        _lib.oracle_moe.argtypes = [f, i, i, i, i, i, f, f, f, f, i, i, f, f]
        _lib.oracle_moe.restype = i
        _lib.oracle_dense_mlp.argtypes = [f, i, i, i, f, f, i, i, f]
        _lib.oracle_dense_mlp.restype = None
        _lib.oracle_shared_combine_f32.argtypes = [f, f, f, f, f, i, i]
        _lib.oracle_shared_combine_f32.restype = None
        _lib.oracle_shared_combine_bf16.argtypes = [f, f, f, f, f, i, i]
        _lib.oracle_shared_combine_bf16.restype = None
        _lib.oracle_silu_and_mul.argtypes = [f, f, i, i, i]
        _lib.oracle_silu_and_mul.restype = None
        _lib.oracle_linear_f32.argtypes = [f, f, f, i, i, i]
        _lib.oracle_linear_f32.restype = None
        _lib.oracle_bf16_round_array.argtypes = [f, f, i64]
        _lib.oracle_bf16_round_array.restype = None
        _lib.oracle_sigmoid.argtypes = [f, f, i64]
        _lib.oracle_sigmoid.restype = None
        _lib.oracle_set_threads.argtypes = [i]
        _lib.oracle_centered_rms_norm.argtypes = [f, f, f, f, f, i, i, ctypes.c_float, i]
        _lib.oracle_centered_rms_norm.restype = None
        _lib.oracle_max_threads.restype = i
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def set_threads(n: int) -> None:
    lib().oracle_set_threads(int(n))


def max_threads() -> int:
    return int(lib().oracle_max_threads())


def bf16_round(a) -> np.ndarray:
    a = _f32(a)
    out = np.empty_like(a)
    lib().oracle_bf16_round_array(_p(a), _p(out), a.size)
    return out


def select_experts(scores, k: int):
    """Returns the K ids or None where the reference bails."""
    s = _f32(scores)
    ids = np.zeros(max(k, 1), dtype=np.int32)
    rc = lib().oracle_select_experts(_p(s), s.size, int(k), _p(ids))
    return None if rc != 0 else ids[:k].tolist()


def route(logits, k: int, normalize: bool = True, want_probabilities: bool = False):
    """logits [T,E] (f32 values) -> (ids [T,K] int32, weights [T,K] f32).

    Raises ValueError with the first rejected token when a row is non-finite,
    as the reference's select_experts does."""
    lg = _f32(logits)
    t, e = lg.shape
    ids = np.zeros((t, k), dtype=np.int32)
    w = np.zeros((t, k), dtype=np.float32)
    probs = np.zeros((t, e), dtype=np.float32) if want_probabilities else None
    rc = lib().oracle_route(_p(lg), t, e, int(k), int(bool(normalize)), _p(ids), _p(w),
                            _p(probs) if probs is not None else None)
    if rc != 0:
        raise ValueError(f"non-finite router row {-1 - rc}")
    if want_probabilities:
        return ids, w, probs
    return ids, w


def plan(ids, num_experts: int):
    ids = _i32(ids)
    t, k = ids.shape
    counts = np.zeros(num_experts, dtype=np.int32)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    slots = np.zeros(t * k, dtype=np.int32)
    lib().oracle_plan(_p(ids), t, k, num_experts, _p(counts), _p(offsets), _p(slots))
    return counts, offsets, slots


def capacity(tokens: int, experts: int, top_k: int, tile_rows: int) -> int:
    return int(lib().oracle_capacity(tokens, experts, top_k, tile_rows))


def dispatch(ids, num_experts: int, tile_rows: int, cap: int | None = None):
    """Padded device layout: (meta[2E+2], offsets[E+1], slots[cap], tiles[cap/M])."""
    ids = _i32(ids)
    t, k = ids.shape
    if cap is None:
        cap = capacity(t, num_experts, k, tile_rows)
    meta = np.zeros(2 * num_experts + 2, dtype=np.int32)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    slots = np.zeros(cap, dtype=np.int32)
    tiles = np.zeros(cap // tile_rows, dtype=np.int32)
    rc = lib().oracle_dispatch(_p(ids), t, k, num_experts, tile_rows, cap,
                               _p(meta), _p(offsets), _p(slots), _p(tiles))
    if rc != 0:
        raise ValueError("capacity too small")
    return meta, offsets, slots, tiles


def moe(x, ids, weights, gate_up, down, act: int = ACT_SILU, bf16: bool = False,
        token_mask=None) -> np.ndarray:
    """Routed experts: x [T,H], ids/weights [T,K], gate_up [E,2I,H], down [E,H,I]."""
    x = _f32(x)
    ids = _i32(ids)
    weights = _f32(weights)
    gate_up = _f32(gate_up)
    down = _f32(down)
    t, h = x.shape
    e, two_i, h2 = gate_up.shape
    assert h2 == h and down.shape == (e, h, two_i // 2)
    k = ids.shape[1]
    out = np.zeros((t, h), dtype=np.float32)
    mask = None
    if token_mask is not None:
        mask = np.ascontiguousarray(token_mask, dtype=np.uint8)
    rc = lib().oracle_moe(_p(x), t, h, two_i // 2, e, k, _p(ids), _p(weights),
                          _p(gate_up), _p(down), int(act), int(bool(bf16)),
                          _p(mask) if mask is not None else None, _p(out))
    if rc != 0:
        raise MemoryError("oracle allocation failed")
    return out


def dense_mlp(x, gate_up, down, act: int = ACT_SILU, bf16: bool = False) -> np.ndarray:
    x = _f32(x)
    gate_up = _f32(gate_up)
    down = _f32(down)
    t, h = x.shape
    i = gate_up.shape[0] // 2
    out = np.zeros((t, h), dtype=np.float32)
    lib().oracle_dense_mlp(_p(x), t, h, i, _p(gate_up), _p(down), int(act), int(bool(bf16)), _p(out))
    return out


def sigmoid(v) -> np.ndarray:
    """f32 1 / (1 + exp(-v)) elementwise, the shared expert's gate."""
    v = _f32(v)
    out = np.empty_like(v)
    lib().oracle_sigmoid(_p(v), _p(out), v.size)
    return out


def shared_combine_f32(x, gate_weight, shared, routed) -> np.ndarray:
    x = _f32(x)
    shared = _f32(shared)
    routed = _f32(routed)
    t, h = x.shape
    out = np.zeros((t, h), dtype=np.float32)
    gw = _f32(gate_weight).reshape(-1) if gate_weight is not None else None
    lib().oracle_shared_combine_f32(_p(x), _p(gw) if gw is not None else None,
                                    _p(shared), _p(routed), _p(out), t, h)
    return out


def shared_combine_bf16(x, gate_weight, shared, routed) -> np.ndarray:
    x = _f32(x)
    shared = _f32(shared)
    routed = _f32(routed)
    gw = _f32(gate_weight).reshape(-1)
    t, h = x.shape
    out = np.zeros((t, h), dtype=np.float32)
    lib().oracle_shared_combine_bf16(_p(x), _p(gw), _p(shared), _p(routed), _p(out), t, h)
    return out


def silu_and_mul(packed, bf16: bool = False) -> np.ndarray:
    packed = _f32(packed)
    rows, two_c = packed.shape
    out = np.zeros((rows, two_c // 2), dtype=np.float32)
    lib().oracle_silu_and_mul(_p(packed), _p(out), rows, two_c // 2, int(bool(bf16)))
    return out


def linear(input_, weight) -> np.ndarray:
    a = _f32(input_)
    b = _f32(weight)
    out = np.zeros((a.shape[0], b.shape[0]), dtype=np.float32)
    lib().oracle_linear_f32(_p(a), _p(b), _p(out), a.shape[0], b.shape[0], a.shape[1])
    return out


def centered_rms_norm(x, weight, eps: float, branch=None, bf16: bool = False):
    """(residual, normalized) of the f32 CPU path; residual is None without a
    branch.  Inputs hold values representable in the storage dtype."""
    x = _f32(x)
    rows, cols = x.reshape(-1, x.shape[-1]).shape
    w = _f32(weight).reshape(-1)
    b = _f32(branch) if branch is not None else None
    out = np.zeros_like(x)
    res = np.zeros_like(x) if b is not None else None
    lib().oracle_centered_rms_norm(_p(x), _p(b) if b is not None else None, _p(w),
                                   _p(res) if res is not None else None, _p(out), rows, cols, float(eps),
                                   int(bool(bf16)))
    return res, out
