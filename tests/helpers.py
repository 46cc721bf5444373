"""Shared comparison helpers for the parity tests."""
import numpy as np


def to_np(x):
    try:
        import torch
        if isinstance(x, torch.Tensor):
            return x.detach().cpu().numpy()
    except ImportError:
        pass
    return np.asarray(x)


def rel_err(got, want) -> float:
    """Norm-relative error max|got - want| / max(max|want|, 1e-30)."""
    g = to_np(got).astype(np.float64).ravel()
    w = to_np(want).astype(np.float64).ravel()
    assert g.shape == w.shape, (g.shape, w.shape)
    if g.size == 0:
        return 0.0
    return float(np.max(np.abs(g - w)) / max(np.max(np.abs(w)), 1e-30))


def psnr(img, ref) -> float:
    a = to_np(img).astype(np.float64)
    b = to_np(ref).astype(np.float64)
    mse = np.mean((a - b) ** 2)
    peak = max(np.max(np.abs(b)), 1e-30)
    if mse == 0:
        return float("inf")
    return float(10.0 * np.log10(peak * peak / mse))
