"""CPU oracle: the model's elementwise algebraic ops (test infrastructure only).

Restates, in float64 NumPy with the reference's roundings to the storage
dtype:

* ``rms_norm`` / ``rms_norm_vjp`` -- algebraic.py:76-83 and the autodiff VJP
  of that expression (no custom VJP in the reference); ``gain=None`` is the
  parameter-free AVN the model uses (model.py:142).
* ``alu_parts`` / ``alu`` / ``alu_vjp`` -- algebraic.py:86-117 (forward with
  the negative-tail form of 1 + u, custom VJP from the cached u, r).
* ``alu_glu`` / ``alu_glu_vjp`` -- the feed-forward product ``gate *
  alu(up)`` of model.py:186-191 and the autodiff VJP of that product, which
  rounds ``dout * gate`` and ``dout * act`` to the storage dtype as the
  unfused bf16 multiplies do.
* ``swiglu`` / ``swiglu_vjp`` -- the standard preset's ``gate * silu(up)``
  (standard.py:12-13), rounding the sigmoid and each product.

Pinned in tests/test_oracle_elementwise.py against the closed form and
finite differences (the reference's own test_components.py:71-78 grid),
torch float64 autograd, and invariants of the norm.
"""

import numpy as np

from .common import F64, cast


def rms_norm(x, gain, eps, dtype):
    """y = cast((x * rsqrt(mean(x^2) + eps)) * gain) (algebraic.py:78-83)."""
    x = np.asarray(x, F64)
    tau = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    y = x * tau
    if gain is not None:
        y = y * np.asarray(gain, F64)
    return cast(y, dtype)


def rms_norm_vjp(x, gain, dy, eps, dtype):
    """(dx, dgain) of rms_norm; dgain is None without a gain.

    With g = dy * gain: dx = tau g - x tau^3 sum(g x) / D (d tau / d x_j =
    -tau^3 x_j / D), dgain = sum over rows of dy * x * tau.
    """
    x = np.asarray(x, F64)
    dy = np.asarray(dy, F64)
    D = x.shape[-1]
    gw = np.ones(D) if gain is None else np.asarray(gain, F64)
    tau = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    g = dy * gw
    dot = np.sum(g * x, axis=-1, keepdims=True)
    dx = tau * g - (tau ** 3) * x * dot / D
    dgain = None if gain is None else cast(np.sum((dy * x * tau).reshape(-1, D), axis=0), "f32")
    return cast(dx, dtype), dgain


def alu_parts(x, beta):
    """(alu(x) unrounded, u, r) in float64 (algebraic.py:86-93)."""
    z = np.asarray(x, F64)
    bz = beta * z
    r = 1.0 / np.sqrt(1.0 + bz * bz)
    u = bz * r
    with np.errstate(divide="ignore", invalid="ignore"):
        one_plus_u = np.where(bz < 0, (r * r) / (1.0 - u), 1.0 + u)
    return 0.5 * z * one_plus_u, u, r


def alu_derivative(u, r):
    """d alu / dx from the cached parts (algebraic.py:108-111)."""
    return 0.5 * (1.0 + u) + 0.5 * u * (r * r)


def alu(x, beta, dtype):
    """alu rounded to the storage dtype (algebraic.py:96-104)."""
    return cast(alu_parts(x, beta)[0], dtype)


def alu_vjp(x, dy, beta, dtype):
    """dx = cast(dy * derivative) (algebraic.py:108-112)."""
    _, u, r = alu_parts(x, beta)
    return cast(np.asarray(dy, F64) * alu_derivative(u, r), dtype)


def alu_glu(gate, up, beta, dtype):
    """out = cast(gate * cast(alu(up))) (model.py:189-191)."""
    act = alu(up, beta, dtype)
    return cast(np.asarray(gate, F64) * act, dtype)


def alu_glu_vjp(gate, up, dout, beta, dtype):
    """(dgate, dup): dgate = cast(dout * act), dup = alu_vjp(up, cast(dout * gate))."""
    act = alu(up, beta, dtype)
    dout = np.asarray(dout, F64)
    dgate = cast(dout * act, dtype)
    gact = cast(dout * np.asarray(gate, F64), dtype)
    return dgate, alu_vjp(up, gact, beta, dtype)


def swiglu(gate, up, dtype):
    """gate * silu(up), silu(x) = x * sigmoid(x) with sigmoid and every product
    rounded to the storage dtype (standard.py:12-13, model.py:186-188)."""
    up = np.asarray(up, F64)
    sg = cast(1.0 / (1.0 + np.exp(-up)), dtype)
    act = cast(up * sg, dtype)
    return cast(np.asarray(gate, F64) * act, dtype)


def swiglu_vjp(gate, up, dout, dtype):
    """(dgate, dup): dgate = cast(dout * act), dup = cast(cast(dout * gate) *
    silu'(up)) with silu' = s + x s (1 - s) unrounded."""
    up = np.asarray(up, F64)
    s = 1.0 / (1.0 + np.exp(-up))
    act = cast(up * cast(s, dtype), dtype)
    dout = np.asarray(dout, F64)
    gact = cast(dout * np.asarray(gate, F64), dtype)
    return cast(dout * act, dtype), cast(gact * (s + up * s * (1.0 - s)), dtype)
