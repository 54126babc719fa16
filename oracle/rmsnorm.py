"""Row-wise RMS normalization, CPU restatement. TEST INFRASTRUCTURE ONLY.

Follows the reference's _rms_forward / _rms_gradient_row (kernels/core_cuda.py:29-75) in
float64 arithmetic with its rounding points to the activation dtype T:
    rstd = 1 / sqrt(mean(x^2) + eps)
    y    = T(T(x * rstd) * T(w))
    g    = T(go * T(w));  gx = rstd * (g - x * rstd^2 * mean(g * x))
    dw   = sum over rows of go * T(x * rstd)
(the reconstruction mode reads y and uses y / T(w) for the normalized values). numpy.
"""

import numpy as np

from .rope import round_to


def forward(x, w, eps, dtype):
    """x [rows, width] float32 holding `dtype` values; w [width] float32 holding the
    weight dtype's values. Returns (y as float32 holding `dtype` values, rstd float64)."""
    x64 = np.asarray(x, dtype=np.float64)
    rstd = 1.0 / np.sqrt((x64 * x64).mean(axis=-1) + eps)
    normalized = round_to((x64 * rstd[:, None]).astype(np.float32), dtype)
    weight = round_to(np.asarray(w, dtype=np.float32), dtype)
    return round_to(normalized.astype(np.float64) * weight, dtype), rstd


def backward(x, w, rstd, go, dtype, *, from_output=False):
    """Input and weight gradients (float64), with the reference's rounding points."""
    x64 = np.asarray(x, dtype=np.float64)
    weight = round_to(np.asarray(w, dtype=np.float32), dtype).astype(np.float64)
    go64 = np.asarray(go, dtype=np.float64)
    g = round_to((go64 * weight).astype(np.float32), dtype).astype(np.float64)
    r = np.asarray(rstd, dtype=np.float64)[:, None]
    if from_output:
        n = x64 / weight
        gx = r * (g - n * (g * n).mean(axis=-1, keepdims=True))
        dw = None
    else:
        gx = r * (g - x64 * (r * r) * (g * x64).mean(axis=-1, keepdims=True))
        dw = (go64 * round_to((x64 * r).astype(np.float32), dtype)).sum(axis=0)
    return gx, dw
