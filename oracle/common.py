"""Shared scalar helpers of the CPU oracle (test infrastructure only).

Elementwise algebra of the reference, restated in float64:

* ``rho_exact``  -- flash.py:76-80, algebraic.py:31-35
* ``rho_fast``   -- flash.py:83-88 (``fast`` branch)
* ``bounded_radical`` / ``tiled_rho`` -- radical.py:13-38 and its per-tile use
  in flash.py:91-92, :172, :229, :349
* ``ipow``       -- flash.py:95-104, algebraic.py:38-51
* ``inv_root``   -- flash.py:107-114, fused_head.py:59-65
* ``root``       -- flash.py:117-123, fused_head.py:39-44
"""

import math

import numpy as np

F64 = np.float64


def rho_exact(x):
    """``(rho(x), r)`` with rho(x)=x+sqrt(1+x^2) stable for x<0 (flash.py:76-80)."""
    x = np.asarray(x, F64)
    rad = 1.0 + x * x
    r = 1.0 / np.sqrt(rad)
    t = np.abs(x) + rad * r
    with np.errstate(divide="ignore"):
        return np.where(x >= 0, t, 1.0 / t), r


def rho_fast(x):
    """``x + rad*rsqrt(rad)`` without the negative-tail reciprocal (flash.py:84-87)."""
    x = np.asarray(x, F64)
    rad = 1.0 + x * x
    r = 1.0 / np.sqrt(rad)
    return x + rad * r, r


def rho(x, fast):
    """Variant rho, flash.py:83-88 (the poly_rho variant: ``tiled_rho``)."""
    return rho_fast(x) if fast else rho_exact(x)


# radical.py:13-16: the reference's float32 polynomial coefficients (constant
# term first) of sqrt(1+t) and 1/sqrt(1+t) on t = x^2 in [0, 1].
SQRT_COEFFICIENTS = (1.0000227161113386, .49927168521732207, -.11935047485233699,
                     .04451694257534509, -.010264432643176741)
RSQRT_COEFFICIENTS = (.9998514827226793, -.49515903732516475, .3364554110926816,
                      -.1841886600636537, .05025262090029994)


def _horner(t, coefficients):
    """radical.py:19-23, with the coefficients rounded to float32 as jnp does."""
    c = [float(np.float32(v)) for v in coefficients]
    p = np.full_like(t, c[-1])
    for v in reversed(c[:-1]):
        p = p * t + v
    return p


def bounded_radical(x):
    """``(rho(x), r)`` by radical.py:26-38: the polynomials when the whole
    array ``x`` has max |x| <= 1 (one lax.cond per call), else the stable
    exact radical."""
    x = np.asarray(x, F64)
    if x.size and np.max(np.abs(x)) <= 1.0:
        t = x * x
        return x + _horner(t, SQRT_COEFFICIENTS), _horner(t, RSQRT_COEFFICIENTS)
    return rho_exact(x)


def tiled_rho(x, fast, poly, bq, bk):
    """The variant rho over score arrays (..., T, T): with ``poly`` the
    bounded radical decided per (bq, bk) block of each (batch, head), as the
    reference's kernels call it on one score tile of one head at a time
    (flash.py:172, :229, :349)."""
    if not poly:
        return rho(x, fast)
    x = np.asarray(x, F64)
    rh = np.empty_like(x)
    r = np.empty_like(x)
    T0, T1 = x.shape[-2:]
    for lead in np.ndindex(*x.shape[:-2]):
        for i in range(0, T0, bq):
            for j in range(0, T1, bk):
                idx = lead + (slice(i, i + bq), slice(j, j + bk))
                rh[idx], r[idx] = bounded_radical(x[idx])
    return rh, r


def ipow(x, n):
    """``x**n`` by binary powering, same multiplication order as flash.py:95-104."""
    n = int(n)
    if n < 1:
        raise ValueError("n must be a positive integer")
    out = None
    base = x
    while n:
        if n & 1:
            out = base if out is None else out * base
        n >>= 1
        if n:
            base = base * base
    return out


def inv_root(l, n):
    """``l**(-1/n)`` for n a power of two via an rsqrt chain (flash.py:107-114)."""
    y = 1.0 / np.sqrt(np.asarray(l, F64))
    k = n // 2
    while k > 1:
        y = y * (1.0 / np.sqrt(y))
        k //= 2
    return y


def root(value, n):
    """``value**(1/n)`` by repeated square roots (flash.py:117-123)."""
    out = float(value)
    while n > 1:
        out = math.sqrt(out)
        n //= 2
    return out


def to_bf16(x):
    """Round-to-nearest-even to bfloat16, returned as float64 values.

    The reference casts with ``astype(jnp.bfloat16)`` (RNE); torch's CPU cast
    is RNE as well. Values first pass through float32 as in the reference,
    whose operands are float32 before the cast.
    """
    import torch
    t = torch.from_numpy(np.ascontiguousarray(np.asarray(x, np.float32)))
    return t.to(torch.bfloat16).to(torch.float64).numpy()


def to_f32(x):
    return np.asarray(x, np.float32).astype(F64)


def cast(x, dtype):
    """Round float64 values to ``dtype`` ("bf16" or "f32") and return float64."""
    if dtype == "bf16":
        return to_bf16(x)
    if dtype == "f32":
        return to_f32(x)
    if dtype == "f64":
        return np.asarray(x, F64)
    raise ValueError(dtype)
