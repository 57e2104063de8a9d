"""Accuracy criterion shared by the GPU parity tests.

fp32: max-abs error <= 1e-5 on unit-scale values, relative beyond |ref| > 1.
16-bit: max-abs error <= 2e-2 (``tol16``) on unit-scale values, relative beyond
|ref| > 1 (where the 16-bit result's own rounding, up to 2^-9 relative, alone
would exceed 2e-2), and mean-relative error <= 1e-2 unless the reference is ~0
everywhere.  The reference is the float64 oracle on the same rounded inputs.
"""

import numpy as np
import torch


def assert_close(actual, expected, dtype, what="", tol16=2e-2):
    actual = actual.detach().double().cpu().numpy()
    err = np.abs(actual - expected)
    if dtype == torch.float32:
        # 1e-5 absolute on unit-scale values, relative beyond |ref| > 1
        scaled = err / np.maximum(1.0, np.abs(expected))
        assert scaled.max() <= 1e-5, f"{what}: scaled max-abs {scaled.max():.3g} (max-abs {err.max():.3g})"
    else:
        # 2e-2 absolute on unit-scale values; relative beyond |ref| > 1, where the
        # 16-bit result's own rounding (up to 2^-9 relative) would exceed 2e-2
        scaled = err / np.maximum(1.0, np.abs(expected))
        assert scaled.max() <= tol16, f"{what}: scaled max-abs {scaled.max():.3g}"
        # mean-relative error; skipped when the reference is ~0 everywhere
        # (e.g. dQ of a single key, which cancels exactly)
        denom = np.abs(expected).mean()
        if denom > 1e-3:
            assert err.mean() / denom <= 1e-2, f"{what}: mean-rel {err.mean() / denom:.3g}"
