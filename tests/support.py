"""Shared helpers for the tests (imported by test modules; not collected)."""

from __future__ import annotations

import numpy as np
import torch

# Tolerances of the attention contract (fp32-accumulated reference result).
OUT_MAX_ABS = 2e-2
OUT_MEAN_ABS = 2e-3
LSE_MAX_ABS = 1e-3


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.float32).cpu().numpy()


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw element bits (int16/int32 view) for bit-exact comparisons."""
    t = t.detach().cpu().contiguous()
    view = {2: torch.int16, 4: torch.int32}[t.element_size()]
    return t.view(view).numpy()


def assert_attention_close(out, lse, ref_out, ref_lse, *, max_abs=OUT_MAX_ABS,
                           mean_abs=OUT_MEAN_ABS, lse_abs=LSE_MAX_ABS, what=""):
    out = np.asarray(out, dtype=np.float64)
    ref_out = np.asarray(ref_out, dtype=np.float64)
    assert np.isfinite(out).all(), f"{what}: non-finite output"
    err = np.abs(out - ref_out)
    assert err.max() <= max_abs, f"{what}: out max-abs {err.max():.3e} > {max_abs}"
    assert err.mean() <= mean_abs, f"{what}: out mean-abs {err.mean():.3e} > {mean_abs}"
    if lse is not None:
        lerr = np.abs(np.asarray(lse, np.float64) - np.asarray(ref_lse, np.float64))
        assert lerr.max() <= lse_abs, f"{what}: lse max-abs {lerr.max():.3e} > {lse_abs}"
    return float(err.max()), float(err.mean())
