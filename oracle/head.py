"""CPU oracle: fused tied-embedding projection + likelihood loss (test infrastructure only).

Restates src/algebraic/kernels/fused_head.py in float64 NumPy:

* ``head_clamp``   -- fused_head.py:273 (= algebraic.likelihood_clamp, algebraic.py:277-283)
* ``forward``      -- fused_head.py:72-117 (per-token statistic and target logit)
* ``telemetry``    -- fused_head.py:219-229 (per-token NLL / target probability, objective)
* ``backward``     -- fused_head.py:120-156, :194-216, :247-254 (scale, dz rounding,
  dh and dE contractions, output casts)
* ``fused_head``   -- fused_head.py:260-275 (validation and dispatch)
* dense checks     -- standard.cross_entropy (standard.py:41-47),
  algebraic.algebraic_likelihood (algebraic.py:223-265),
  evaluation.logprob_from_logits (evaluation.py:13-23)
"""

import numpy as np

from .common import F64, cast, inv_root, ipow, rho_exact, root


def head_clamp(vocab, n):
    """fused_head.py:273 / algebraic.py:277-283."""
    return 0.25 * root(1e38 / vocab, n)


def _logits(h, e):
    return np.asarray(h, F64) @ np.asarray(e, F64).T


def forward(h, e, targets, *, kind, n, c, clamp, stat_dtype="f32"):
    """(stat, zt) per token; e is the embedding already cast to h's dtype."""
    z = _logits(h, e)
    N, V = z.shape
    zt = z[np.arange(N), targets]
    if kind == "ce":
        m = z.max(-1)
        stat = m + np.log(np.exp(z - m[:, None]).sum(-1))
    else:
        x = np.minimum(z * (1.0 / c), clamp)
        rad = 1.0 + x * x
        w = ipow(x + rad * (1.0 / np.sqrt(rad)), n)
        stat = inv_root(w.sum(-1), n)
    return cast(stat, stat_dtype), cast(zt, stat_dtype)


def telemetry(stat, zt, *, kind, n, c, clamp):
    """fused_head.py:219-229: (telemetry, objective)."""
    stat, zt = np.asarray(stat, F64), np.asarray(zt, F64)
    if kind == "ce":
        nll = stat - zt
        return nll, float(np.mean(nll))
    x = np.minimum(zt / c, clamp)
    pt = ipow(rho_exact(x)[0] * stat, n)
    return pt, float(np.mean(1.0 - pt))


def backward(h, e, targets, stat, g_obj, *, kind, n, c, clamp, dtype, embed_dtype="f32"):
    """(dh, dE) following fused_head.py:120-156, :194-216, :247-254."""
    z = _logits(h, e)
    N, V = z.shape
    slope = 1.0 if kind == "ce" else n / c
    scale = g_obj * (slope / N)
    if dtype != "f64":
        scale = float(np.float32(scale))
    y = np.zeros_like(z)
    y[np.arange(N), targets] = 1.0
    stat = np.asarray(stat, F64)[:, None]
    if kind == "ce":
        dz = np.exp(z - stat) - y
    else:
        x = np.minimum(z * (1.0 / c), clamp)
        rad = 1.0 + x * x
        r = 1.0 / np.sqrt(rad)
        p = ipow((x + rad * r) * stat, n)
        dz = (p - y) * r
    dzb = cast(dz * scale, dtype)
    dh = dzb @ np.asarray(e, F64)
    de = dzb.T @ np.asarray(h, F64)
    return cast(dh, dtype), cast(de, embed_dtype)


def fused_head(h, embed, targets, *, kind="ce", n=16, c=16.0, dtype="bf16",
               embed_dtype="f32", g_obj=None):
    """fused_head.py:260-275 -> ((objective, telemetry), grads or None)."""
    if kind not in ("ce", "alg_ce"):
        raise ValueError(kind)
    if kind == "alg_ce" and (n & (n - 1)):
        raise ValueError("n must be a power of two")
    V = np.asarray(embed).shape[0]
    clamp = head_clamp(V, n) if kind == "alg_ce" else 0.0
    e = cast(embed, dtype)                                      # fused_head.py:168
    targets = np.asarray(targets, np.int64)
    stat, zt = forward(h, e, targets, kind=kind, n=n, c=c, clamp=clamp,
                       stat_dtype="f64" if dtype == "f64" else "f32")
    tel, obj = telemetry(stat, zt, kind=kind, n=n, c=c, clamp=clamp)
    grads = None
    if g_obj is not None:
        grads = backward(h, e, targets, stat, g_obj, kind=kind, n=n, c=c, clamp=clamp,
                         dtype=dtype, embed_dtype=embed_dtype)
    return (obj, tel), grads


def dense_alg_logprob(z, targets, n, c):
    """evaluation.py:13-23 for head="alg_ce": log_softmax(n asinh(z/c))[t]."""
    a = n * np.arcsinh(np.asarray(z, F64) / c)
    a = a - a.max(-1, keepdims=True)
    lse = np.log(np.exp(a).sum(-1))
    return a[np.arange(len(targets)), targets] - lse


def dense_ce(z, targets):
    """standard.py:41-47: (mean NLL, per-token NLL)."""
    z = np.asarray(z, F64)
    m = z.max(-1, keepdims=True)
    lse = (m + np.log(np.exp(z - m).sum(-1, keepdims=True)))[:, 0]
    nll = lse - z[np.arange(len(targets)), targets]
    return float(nll.mean()), nll
