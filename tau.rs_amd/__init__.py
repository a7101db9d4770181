"""tau.rs_amd: MI355X-native MoE expert-FFN path (HIP for gfx950 behind a C ABI).

Load as a package named ``tau_rs_amd`` (the directory name holds a dot); see
``tests/conftest.py`` and ``__graft_entry__.py``.
"""
from . import checkpoint, ffi, inputs, norm, sparse_moe  # noqa: F401
from .norm import CenteredRmsNorm, moe_feed_forward  # noqa: F401
from .sparse_moe import (MoePrefillRunner, MoePrefillTile, SharedExpertConfig, SparseMoeBlock,  # noqa: F401
                         SparseMoeConfig, moe_prefill_capacity)
