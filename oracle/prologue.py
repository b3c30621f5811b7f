"""CPU oracle: the model block's attention prologue (test infrastructure only).

Restates model.py:166-174 for 64-wide heads: the (B, T, H, D) projections
RMS-normalised over D with a gain (the QK-norm oracle, algebraic.py:76-83),
rotated by the rotate-half product (algebraic.py:172-179) with the tables and
every product and sum rounded to the model dtype as the reference's ops round,
and laid out as (B, H, T, D); and the VJP of that chain (rotation by the
transposed matrix with the same roundings, then the QK-norm VJP). Pinned in
tests/test_oracle_model.py against complex multiplication and torch float64
autograd.
"""

import numpy as np

from .common import F64, cast
from . import qknorm as OQ


def _rot_tables(cos, sin, dtype):
    return cast(np.asarray(cos, F64), dtype)[None, :, None, :], \
        cast(np.asarray(sin, F64), dtype)[None, :, None, :]


def forward(x, gain, cos, sin, eps, dtype):
    """x: (B, T, H, D) projections -> (B, H, T, D); gain None: no norm;
    cos None: no rotation."""
    x = np.asarray(x, F64)
    y = OQ.forward(x, gain, eps, dtype) if gain is not None else x
    if cos is not None:
        c, s = _rot_tables(cos, sin, dtype)
        h = y.shape[-1] // 2
        y1, y2 = y[..., :h], y[..., h:]
        y = np.concatenate([cast(cast(y1 * c, dtype) - cast(y2 * s, dtype), dtype),
                            cast(cast(y1 * s, dtype) + cast(y2 * c, dtype), dtype)], -1)
    return np.transpose(y, (0, 2, 1, 3))


def backward(x, gain, cos, sin, dout, eps, dtype):
    """(dx in (B, T, H, D), dgain or None) for dout in (B, H, T, D)."""
    d = np.transpose(np.asarray(dout, F64), (0, 2, 1, 3))
    if cos is not None:
        c, s = _rot_tables(cos, sin, dtype)
        h = d.shape[-1] // 2
        d1, d2 = d[..., :h], d[..., h:]
        d = np.concatenate([cast(cast(d1 * c, dtype) + cast(d2 * s, dtype), dtype),
                            cast(cast(d2 * c, dtype) - cast(d1 * s, dtype), dtype)], -1)
    if gain is None:
        return d, None
    return OQ.backward(np.asarray(x, F64), gain, d, eps, dtype)
