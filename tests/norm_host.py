"""Host-side helpers shared by the norm oracle checks and the GPU norm tests:
the reference tests' input pattern, the f64 closed form and the comparison
rule of crates/models/src/components/cuda/rms_norm/tests/residual/support.rs."""
import numpy as np
import torch


def patterned(count, phase):
    """The reference tests' input pattern (residual/support.rs:44-55)."""
    i = np.arange(count, dtype=np.int64)
    return (((i * 17 + phase) % 127).astype(np.float32) / np.float32(37.0) - np.float32(1.7)).astype(np.float32)


def to_dtype(a, bf16):
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    return t.to(torch.bfloat16).float().numpy() if bf16 else t.numpy()


def f64_norm(rows, weight, eps):
    """test_support.rs:5-27: f64 reduction, centered scale 1 + w rounded in f32."""
    rows64 = rows.astype(np.float64)
    inv = 1.0 / np.sqrt((rows64 ** 2).sum(axis=-1, keepdims=True) / rows.shape[-1] + np.float64(eps))
    return (rows64 * inv * (np.float32(1.0) + weight.astype(np.float32)).astype(np.float64)).astype(np.float32)


def assert_close(actual, expected, bf16):
    """residual/support.rs:22-42: BF16 within one ulp, f32 1e-6 + 2e-6|b|."""
    a = np.asarray(actual, np.float32).ravel()
    b = np.asarray(expected, np.float32).ravel()
    assert np.all(np.isfinite(a)) and np.all(np.isfinite(b))
    if bf16:
        ab = torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().astype(np.int32)
        bb = torch.from_numpy(b).to(torch.bfloat16).view(torch.int16).numpy().astype(np.int32)
        assert np.max(np.abs(ab - bb)) <= 1
    else:
        assert np.all(np.abs(a - b) <= 1e-6 + 2e-6 * np.abs(b))
