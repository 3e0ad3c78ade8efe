"""Shared test utilities: GPU detection, bf16 <-> fp32 exact conversion,
and the numeric tolerance bars of the path."""

import numpy as np
import torch

# Output tolerances (bf16: max-abs / mean-abs; fp32: max-abs).
BF16_MAX_ABS = 2e-2
BF16_MEAN_ABS = 2e-3
F32_MAX_ABS = 1e-4


def gpu():
    return torch.cuda.is_available()


def np32(t: torch.Tensor) -> np.ndarray:
    """Exact fp32 numpy copy (bf16 widens exactly)."""
    return t.detach().float().cpu().numpy()


def assert_close_out(got: np.ndarray, want: np.ndarray, dtype, mask=None, what="output"):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    if mask is not None:
        got, want = got[mask], want[mask]
    err = np.abs(got - want)
    assert np.isfinite(got).all(), f"{what}: non-finite values"
    if dtype == torch.bfloat16:
        assert err.max() <= BF16_MAX_ABS, f"{what}: max-abs {err.max():.3e} > {BF16_MAX_ABS}"
        assert err.mean() <= BF16_MEAN_ABS, f"{what}: mean-abs {err.mean():.3e} > {BF16_MEAN_ABS}"
    else:
        assert err.max() <= F32_MAX_ABS, f"{what}: max-abs {err.max():.3e} > {F32_MAX_ABS}"
    return err.max(), err.mean()
