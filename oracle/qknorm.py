"""CPU oracle: QK RMS normalisation with a learned gain (test infrastructure only).

Restates ``algebraic.rms_norm`` (algebraic.py:76-83), the custom VJP of
``qk_rms_norm`` (qk_norm.py:29-59: native input VJP, tiled gain reduction)
and its validation (qk_norm.py:62-76), in float64 NumPy.
"""

import numpy as np

from .common import F64, cast


def forward(x, gain, eps, dtype):
    """y = x * rsqrt(mean(x^2) + eps) * gain, rounded to x's dtype (algebraic.py:78-83)."""
    x = np.asarray(x, F64)
    tau = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return cast(x * tau * np.asarray(gain, F64), dtype)


def backward(x, gain, dy, eps, dtype):
    """(dx, dgain): input VJP of rms_norm (qk_norm.py:42-43) and the gain
    reduction sum_rows dy*x*tau (qk_norm.py:20-26, :55)."""
    x = np.asarray(x, F64)
    g = np.asarray(gain, F64)
    dy = np.asarray(dy, F64)
    D = x.shape[-1]
    tau = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    dot = np.sum(dy * g * x, axis=-1, keepdims=True)
    dx = tau * g * dy - (tau ** 3) * x * dot / D
    dgain = np.sum((dy * x * tau).reshape(-1, D), axis=0)
    return cast(dx, dtype), cast(dgain, "f32")


def validate(shape, D, gain_shape, x_dtype, gain_dtype, rows, block, eps):
    """Error conditions of qk_norm.py:68-75 (returns the message or None)."""
    if len(shape) < 2 or D != 64 or tuple(gain_shape) != (64,):
        return "QK RMS kernel needs D=64 and a one-dimensional gain"
    if x_dtype not in ("bf16", "f32") or gain_dtype != "f32":
        return "QK RMS kernel needs float32/BF16 input and float32 gain"
    if block < 8 or block % 8 or rows % block:
        return "QK RMS row count must be divisible by a block aligned to eight rows"
    if eps <= 0:
        return "QK RMS epsilon must be positive"
    return None
