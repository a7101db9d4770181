"""Host-side checks that need no GPU: the C ABI loads and exports every
declared symbol, launchers reject bad arguments before touching the device,
and the Python mirror of the reference's config types behaves like it."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "tau_moe.h")).read()
    return sorted(set(re.findall(r"\b(tau_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol(tau):
    lib = tau.ffi.lib()
    syms = header_symbols()
    assert len(syms) >= 20
    for name in syms:
        assert hasattr(lib, name), name
    assert set(syms) == set(tau.ffi.EXPORTS)
    assert lib.tau_moe_build_target() == b"gfx950"


def test_capacity_and_workspace_queries(tau):
    assert tau.ffi.capacity(1, 256, 8, 16) == 128  # prefill/tests.rs:127
    assert tau.moe_prefill_capacity(0) is None
    assert tau.moe_prefill_capacity(1) == 128
    sizes = tau.ffi.workspace_bytes(64, 2048, 768, 128, 8, 16)
    cap = tau.ffi.capacity(64, 128, 8, 16)
    assert sizes == [64 * 16 * 4, 258 * 4, 129 * 4, cap * 4, cap // 16 * 4, cap * 768 * 2, 64 * 8 * 2048 * 2]


def test_launchers_reject_invalid_arguments_without_a_device(tau):
    L = tau.ffi.lib()
    null = None
    assert L.tau_launch_moe_routing_fp32(null, null, 4, null) == 1
    assert L.tau_launch_moe_prefill_dispatch(null, null, null, null, null, 4, 128, 16, null) == 1
    assert L.tau_launch_moe_prefill_combine(null, null, null, 1, 8, null) == 1
    assert L.tau_launch_silu_and_mul(null, null, 1, 1, 1, null) == 1
    assert L.tau_launch_moe_shared_combine(null, null, null, null, null, 1, 8, null) == 1
    assert L.tau_launch_linear_bf16_fp32(null, null, null, 1, 1, 1, null) == 1
    assert L.tau_launch_moe_routing_ex(null, 1, null, 4, 128, 8, null) == 1
    # fused decode reports argument errors as -1 (fused_bf16_moe_decode.cu:63-66)
    assert L.tau_launch_fused_bf16_moe_decode(*([null] * 13), 2048, 768, 256, 8, null, null, null, null) == -1
    # non-null placeholders with invalid shapes are still rejected on the host
    dummy = ctypes.c_void_p(16)
    assert L.tau_launch_moe_routing_ex(dummy, 1, dummy, 4, 1025, 8, null) == 1  # E > 512
    assert L.tau_launch_moe_routing_ex(dummy, 1, dummy, 4, 128, 0, null) == 1
    assert L.tau_launch_moe_routing_ex(dummy, 1, dummy, 4, 8, 9, null) == 1     # K > E
    assert L.tau_launch_moe_prefill_dispatch(dummy, dummy, dummy, dummy, dummy, 4, 127, 16, null) == 1  # capacity
    assert L.tau_moe_prefill_capacity(1, 256, 8, 48) == -1
    # routing flags: only TAU_MOE_ROUTE_RAW_WEIGHTS may be OR-ed into the dtype
    assert L.tau_launch_moe_routing_ex(dummy, 1 | 0x200, dummy, 4, 128, 8, null) == 1
    assert L.tau_launch_moe_routing_ex(dummy, 2 | 0x100, dummy, 4, 128, 8, null) == 1
    # decode projections: tokens <= 64, E <= 256, plan buffers for the down projection
    assert L.tau_launch_moe_decode_projection_ex(*([dummy] * 8), 65, 2048, 768, 128, 8, 4096, 0, 1, null, null) == 1
    assert L.tau_launch_moe_decode_projection_ex(*([dummy] * 8), 64, 2048, 768, 512, 8, 4096, 0, 1, null, null) == 1
    assert L.tau_launch_moe_decode_projection_ex(dummy, dummy, dummy, null, null, null, null, dummy,
                                                 64, 2048, 768, 128, 8, 4096, 1, 1, null, null) == 1


def test_sparse_moe_config_validation_messages(tau):
    C = tau.SparseMoeConfig
    C(2, 2, 2, 1, shared_expert=tau.SharedExpertConfig(2)).validate()
    with pytest.raises(ValueError, match="cannot exceed"):
        C(2, 2, 2, 3).validate()
    with pytest.raises(ValueError, match="non-zero"):
        C(0, 2, 2, 1).validate()
    with pytest.raises(ValueError, match="shared-expert"):
        C(2, 2, 2, 1, shared_expert=tau.SharedExpertConfig(0)).validate()


def test_prefill_tile_parse_and_validate(tau):
    T = tau.MoePrefillTile
    assert T.parse("16,64,64,4,1").values() == [16, 64, 64, 4, 1]
    assert str(T.parse("32,32,32,2,2")) == "32,32,32,2,2"
    assert T().values() == [16, 16, 16, 1, 1]
    for bad in ["16,64,64,4", "16,64,64,4,1,1", "a,b,c,d,e", "24,64,64,4,1", "16,64,64,3,1"]:
        with pytest.raises(ValueError):
            T.parse(bad)


def test_frag16_host_orders_agree_and_match_spot_values():
    import numpy as np
    from frag16_host import frag16_loop, frag16_permute
    rng = np.random.default_rng(5)
    for shape in [(2, 32, 128), (48, 64), (1, 16, 64)]:
        w = rng.integers(0, 1 << 16, size=shape, dtype=np.uint16)
        a, b = frag16_loop(w), frag16_permute(w)
        np.testing.assert_array_equal(a, b)
        assert sorted(a.ravel().tolist()) == sorted(w.ravel().tolist())  # a permutation
    # Spot values fixed by the definition, independent of both restatements:
    # element (row, col) of a [n, k] matrix at flat index row * k + col.
    n, k = 32, 128
    w = np.arange(n * k, dtype=np.int64).reshape(n, k)
    p = frag16_loop(w).reshape(-1, 8)
    assert p[0].tolist() == list(range(0, 8))                      # row 0, cols 0..7
    assert p[1].tolist() == list(range(k, k + 8))                  # lane 1 -> row 1
    assert p[16].tolist() == list(range(8, 16))                    # lane 16 -> cols 8..15
    assert p[64].tolist() == list(range(32, 40))                   # next 32-wide K chunk
    assert p[(k // 32) * 64].tolist() == list(range(16 * k, 16 * k + 8))  # next 16-row band


def test_frag16_entry_points_reject_unsupported_shapes(tau):
    L = tau.ffi.lib()
    d = ctypes.c_void_p(16)
    e = ctypes.c_void_p(4096)
    assert L.tau_moe_pack_weights(d, e, 2, 24, 128, None) == 1   # rows % 16
    assert L.tau_moe_pack_weights(d, e, 2, 32, 96, None) == 1    # columns % 64
    assert L.tau_moe_pack_weights(d, d, 2, 32, 128, None) == 1   # in place
    args = [d] * 13
    # hidden 96 is not a whole number of 64-wide K steps: frag16 rejected
    assert L.tau_launch_moe_prefill_ex(d, d, 1, d, d, *args[:8], 64, 96, 128, 8, 2, 16, 4096, 1, None, None,
                                       None) == 1
    # unknown layout code
    assert L.tau_launch_moe_prefill_ex(d, d, 1, d, d, *args[:8], 64, 128, 128, 8, 2, 16, 4096, 7, None, None,
                                       None) == 1
    assert L.tau_launch_moe_grouped_gemm_ex(*([d] * 7), 64, 96, 128, 8, 2, 16, 4096, 0, 1, None, None) == 1


def test_routing_flag_bits_are_validated_on_every_entry_point(tau):
    """Only TAU_MOE_ROUTE_RAW_WEIGHTS (0x100) may be OR-ed into logits_dtype:
    any other bit, or a dtype other than 0/1, is rejected before a launch."""
    L = tau.ffi.lib()
    d = ctypes.c_void_p(16)
    for bad in (2, 0x200, 0x101 | 0x400, -1):
        assert L.tau_launch_moe_routing_ex(d, bad, d, 4, 128, 8, None) == 1
        assert L.tau_launch_moe_routing_shared_ex(d, bad, d, 4, 128, 8, None) == 1
        assert L.tau_launch_moe_prefill_dispatch_ex(d, bad, d, d, d, d, d, 4, 128, 8, 16, 4096, None) == 1
        assert L.tau_launch_moe_prefill_ex(d, d, bad, d, d, *([d] * 8), 64, 2048, 768, 128, 8, 16, 4096, 0, None,
                                           None, None) == 1
    assert tau.ffi.ROUTE_RAW_WEIGHTS == 0x100


def test_unnormalised_config_is_accepted_by_the_host_mirror(tau):
    cfg = tau.SparseMoeConfig(64, 64, 8, 2, normalize_selected_weights=False)
    cfg.validate()  # the reference honours the flag (routing.rs:198-202); so does the HIP path
