"""Small helpers shared by the test modules."""

import numpy as np


def rel_err(a, b) -> float:
    """Normwise relative error max|a - b| / max(max|b|, 1e-30), one number per tensor."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    if a.shape != b.shape:
        raise AssertionError(f"shape mismatch {a.shape} vs {b.shape}")
    if b.size == 0:
        return 0.0
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def to_np(t):
    """torch tensor (any device / dtype) -> float64 numpy array."""
    import torch

    return t.detach().to("cpu", torch.float64).numpy()
