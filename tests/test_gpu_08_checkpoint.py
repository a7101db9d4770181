"""A block loaded from a checkpoint equals the block built from the same
tensors directly, bit for bit (run with -m gpu)."""
import numpy as np
import pytest
import torch

from test_checkpoint import E, H, P, config, tensors, write_individual, write_packed

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)


@pytest.mark.parametrize("layout", ["individual", "packed"])
def test_loaded_block_matches_direct_block(tau, tmp_path, layout):
    print(f"[checkpoint block] {layout}", flush=True)
    t = tensors(1)
    paths = (write_individual if layout == "individual" else write_packed)(tmp_path, t)
    cfg = config(tau)
    blk = tau.checkpoint.load_sparse_moe_block(paths, P, cfg)
    d = {k: v.cuda() for k, v in t.items()}
    ref = tau.SparseMoeBlock(cfg, torch.cat([d["gate"], d["up"]], 1), d["down"], torch.cat([d["sg"], d["su"]], 0),
                             d["sd"], d["sgate"], router_weight=d["router"])
    x = torch.randn(24, H, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).cuda()
    a, b = blk.forward(x), ref.forward(x)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(a.view(torch.int16).cpu().numpy(), b.view(torch.int16).cpu().numpy())
