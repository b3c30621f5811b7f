"""CPU oracle: causal asinh-power / softmax flash attention (test infrastructure only).

Restates the reference's numerics densely in float64 NumPy, rounding to the
input dtype exactly where the reference rounds:

* ``Variant`` / ``make_variant``    -- flash.py:59-73, :732-760
* ``guard_in_range``                -- flash.py:834-849 (range guard predicate)
* ``forward``                       -- flash.py:189-284 (generic kernel) and
  head_resident.py:24-93 (whole-head kernel); tile order is immaterial in
  exact arithmetic, so the oracle forms whole rows at once
* ``backward``                      -- flash.py:333-361 (``_tile_grads``),
  :630-638 (``di``), :430-432 / head_resident.py:130-132 (slope ``n``),
  rounding points flash.py:461 and head_resident.py:124
* ``sink_mass_and_slope``           -- flash.py:694-705, used at :721-723
* ``flash_attention``               -- flash.py:763-857 (public wrapper:
  q pre-scale and its rounding :833, sink division :825-830, guard dispatch)
* ``dense_asinh_attention``         -- algebraic.py:186-216
* ``dense_softmax_attention``       -- standard.py:24-38

Pinned in tests/test_oracle.py against the softmax-of-compressed-logits
identity (test_components.py:28-41), float64 torch autograd, finite
differences and the reference's known-answer constants.
"""

import math
from typing import NamedTuple, Optional

import numpy as np

from .common import F64, bounded_radical, cast, inv_root, ipow, rho, rho_exact, root, tiled_rho

NEG = -1e4  # flash.py:55 -- finite "minus infinity" of the shifted kernels


class Variant(NamedTuple):
    """flash.py:59-73 (schedule flags omitted: they do not change numerics)."""
    kind: str
    n: int = 16
    shift: bool = True
    fast_rho: bool = False
    clamp: float = 0.0
    inv_stat: bool = False
    compact_stat: bool = False
    poly_rho: bool = False
    bounded_scores: bool = False
    precise_output: bool = False


def make_variant(kind, n=16, c=16.0, seq_len=2048, shift=None, fast_rho=None,
                 inv_stat=None, compact_stat=True, poly_rho=False):
    """flash.py:732-760."""
    if kind == "softmax":
        return Variant("softmax", compact_stat=bool(compact_stat))
    if kind != "asinh":
        raise ValueError(f"unknown attention kernel: {kind}")
    if n < 2 or n & (n - 1):
        raise ValueError("asinh kernel needs n to be a power of two")
    if not math.isfinite(c) or c <= 0:
        raise ValueError("asinh scale c must be positive and finite")
    t = root(1e37 / (seq_len + 1), n)
    clamp = 0.5 * (t - 1.0 / t)
    if shift is None:
        shift = clamp < 20.0
    if fast_rho is None:
        fast_rho = True
    if inv_stat is None:
        inv_stat = not shift
    if inv_stat and shift:
        raise ValueError("inverse-denominator statistic requires shift=False")
    if poly_rho and (shift or n != 16):
        raise ValueError("bounded radical approximation requires shift=False and n=16")
    return Variant("asinh", int(n), bool(shift), bool(fast_rho), float(clamp),
                   bool(inv_stat), bool(compact_stat), bool(poly_rho))


def guard_bounds(var, T, has_sink):
    """(bound, vmax) of the range guard, flash.py:840, :848."""
    bound = min(16.0, var.clamp / 2)
    vmax = min(1e8, 1e37 / ((T + int(has_sink)) * (2 * bound + 1) ** var.n))
    return bound, vmax


def guard_in_range(q_scaled, k, v, sink, var, has_sink):
    """flash.py:841-849, reductions in float32 as in the reference."""
    T = q_scaled.shape[-2]
    bound, vmax = guard_bounds(var, T, has_sink)
    q2 = np.max(np.sum(np.asarray(q_scaled, np.float32) ** 2, axis=-1, dtype=np.float32))
    k2 = np.max(np.sum(np.asarray(k, np.float32) ** 2, axis=-1, dtype=np.float32))
    ok = bool(np.float32(q2) * np.float32(k2) <= np.float32((bound / 1.01) ** 2))
    if has_sink:
        ok = ok and bool(np.max(np.abs(np.asarray(sink, np.float32))) <= np.float32(bound / 1.01))
    ok = ok and bool(np.max(np.abs(np.asarray(v, np.float32))) <= np.float32(vmax))
    return ok


def low_high(var):
    """The guarded pair of variants, flash.py:850-852."""
    low = var._replace(shift=False, inv_stat=True, bounded_scores=True)
    high = var._replace(shift=True, inv_stat=False, fast_rho=False,
                        bounded_scores=False, precise_output=True)
    return low, high


def _stat_dtype(dtype):
    """Statistics and precise outputs are float32 in the reference (float64 in
    the oracle's exact mode ``dtype="f64"``)."""
    return "f64" if dtype == "f64" else "f32"


def _causal(T):
    return np.tril(np.ones((T, T), bool))


def _scores(qs, k):
    return np.einsum("bhqd,bhkd->bhqk", np.asarray(qs, F64), np.asarray(k, F64))


def forward(qs, k, v, sink, var, has_sink, dtype, block=(512, 512)):
    """Kernel forward on pre-scaled ``qs``; returns ``(o, o_residual, stat)``.

    ``sink`` is the (H,) kernel-unit sink (already divided by ``c``).
    flash.py:197-284 / head_resident.py:24-93:
      * softmax: running max ``m`` (init sink or NEG), ``p = exp(s - m)``,
        stat ``m + log l``;
      * asinh unshifted: ``p = rho(x)^n`` with ``x = s`` (bounded scores) or
        ``min(s, clamp)``, ``l`` seeded with the sink weight, stat ``1/l``
        (inv_stat) or ``l^(-1/n)``;
      * asinh shifted: ``p = (rho(x) rho(-m))^n`` with the exact rho for the
        shift, stat ``rho(-m) l^(-1/n)``.
    ``p`` is rounded to the value dtype before the PV product
    (flash.py:233/258, head_resident.py:86); the output is rounded to the
    input dtype unless ``precise_output`` (flash.py:322).
    """
    B, H, T, D = qs.shape
    s = _scores(qs, k)
    mask = _causal(T)[None, None]
    b = np.asarray(sink, F64)[None, :, None] if has_sink else None   # (1,H,1)
    if var.kind == "softmax":
        m = np.max(np.where(mask, s, -np.inf), axis=-1)
        if has_sink:
            m = np.maximum(m, b)
        p = np.where(mask, np.exp(s - m[..., None]), 0.0)
        l = p.sum(-1) + (np.exp(b - m) if has_sink else 0.0)
        stat = m + np.log(l)
    elif not var.shift:
        x = s if var.bounded_scores else np.minimum(s, var.clamp)
        bq, bk = min(block[0], T), min(block[1], T)
        p = np.where(mask, ipow(tiled_rho(x, var.fast_rho, var.poly_rho, bq, bk)[0], var.n), 0.0)
        l = p.sum(-1)
        if has_sink:
            xb = b if var.bounded_scores else np.minimum(b, var.clamp)
            # one head's sink fills the l_sc tile (flash.py:201-205)
            rb = (np.stack([bounded_radical(xb[:, h])[0] for h in range(H)], axis=1)
                  if var.poly_rho else rho(xb, var.fast_rho)[0])
            l = l + ipow(rb, var.n)
        stat = 1.0 / l if var.inv_stat else inv_root(l, var.n)
    else:
        m = np.max(np.where(mask, s, -np.inf), axis=-1)
        if has_sink:
            m = np.maximum(m, b)
        shift = rho_exact(-m)[0]
        p = np.where(mask, ipow(rho(np.where(mask, s, 0.0), var.fast_rho)[0]
                                * shift[..., None], var.n), 0.0)
        l = p.sum(-1)
        if has_sink:
            l = l + ipow(rho_exact(b)[0] * shift, var.n)
        stat = shift * inv_root(l, var.n)
    pv = np.einsum("bhqk,bhkd->bhqd", cast(p, dtype), np.asarray(v, F64))
    o_full = pv / l[..., None]
    o = cast(o_full, dtype)
    o_res = cast(o_full, _stat_dtype(dtype)) if var.precise_output else o
    return o, o_res, cast(stat, _stat_dtype(dtype))


def sink_mass_and_slope(sink, stat, var):
    """Per-row sink probability (B,H,T) and d(logit)/d(sink), flash.py:694-705."""
    sink = np.asarray(sink, F64)
    if var.kind == "softmax":
        return np.exp(sink[None, :, None] - stat), np.ones_like(sink)
    bb = np.minimum(sink, var.clamp) if (not var.shift and not var.bounded_scores) else sink
    rh, r = bounded_radical(bb) if var.poly_rho else rho_exact(bb)   # over all heads at once
    mass = (ipow(rh[None, :, None], var.n) * stat if var.inv_stat
            else ipow(rh[None, :, None] * stat, var.n))
    slope = var.n * r
    if not var.shift and not var.bounded_scores:
        slope = np.where(sink < var.clamp, slope, 0.0)
    return mass, slope


def backward(qs, k, v, sink, o_res, stat, do, var, has_sink, dtype, block=(512, 512)):
    """Kernel VJP w.r.t. (qs, k, v, sink); flash.py:333-361, :630-638, :718-726.

    ``dq`` is w.r.t. the pre-scaled query (the wrapper applies ``scale``).
    """
    B, H, T, D = qs.shape
    do = np.asarray(do, F64)
    di = np.sum(do * np.asarray(o_res, F64), axis=-1)              # flash.py:633
    s = _scores(qs, k)
    mask = _causal(T)[None, None]
    stat_ = np.asarray(stat, F64)[..., None]
    if var.kind == "softmax":
        p = np.exp(np.where(mask, s, -np.inf) - stat_)
        r = None
    else:
        if not var.shift:
            x = s if var.bounded_scores else np.minimum(s, var.clamp)
        else:
            x = np.where(mask, s, 0.0)
        bq, bk = min(block[0], T), min(block[1], T)
        rh, r = tiled_rho(x, var.fast_rho, var.poly_rho, bq, bk)
        p = ipow(rh, var.n) * stat_ if var.inv_stat else ipow(rh * stat_, var.n)
    p = np.where(mask, p, 0.0)
    dp = np.einsum("bhqd,bhkd->bhqk", do, np.asarray(v, F64))
    ds = p * (dp - di[..., None])
    if r is not None:
        ds = ds * r
        if not var.shift and not var.bounded_scores:
            ds = np.where(s < var.clamp, ds, 0.0)
    ds = np.where(mask, ds, 0.0)
    slope = 1.0 if var.kind == "softmax" else float(var.n)
    pb, dsb = cast(p, dtype), cast(ds, dtype)
    dv = np.einsum("bhqk,bhqd->bhkd", pb, do)
    dk = np.einsum("bhqk,bhqd->bhkd", dsb, np.asarray(qs, F64)) * slope
    dq = np.einsum("bhqk,bhkd->bhqd", dsb, np.asarray(k, F64)) * slope
    if has_sink:
        mass, slope_b = sink_mass_and_slope(sink, stat, var)
        dsink = -np.sum(mass * di, axis=(0, 2)) * slope_b
    else:
        dsink = np.zeros(H)
    return cast(dq, dtype), cast(dk, dtype), cast(dv, dtype), dsink, di


class Result(NamedTuple):
    o: np.ndarray
    stat: np.ndarray
    variant: Variant
    in_range: Optional[bool]
    grads: Optional[tuple]


def flash_attention(q, k, v, sink_logit=None, *, kind="softmax", n=16, c=16.0,
                    shift=None, fast_rho=None, inv_stat=None, compact_stat=True,
                    poly_rho=False, range_guard=False, dtype="f32", do=None, block=512,
                    block_q=None, block_k=None):
    """Public wrapper semantics, flash.py:793-857, plus its custom VJP.

    Inputs are float64 arrays holding values representable in ``dtype``
    ("bf16" or "f32"). With ``do`` the VJP ``(dq, dk, dv, dsink_logit)`` is
    returned as well; ``dsink_logit`` has ``sink_logit``'s shape.
    """
    q, k, v = (np.asarray(a, F64) for a in (q, k, v))
    B, H, T, D = q.shape
    tiles = (block_q or block, block_k or block)   # Pallas score tiles (poly_rho's cond)
    var = make_variant(kind, n, c, T, shift, fast_rho, inv_stat, compact_stat, poly_rho)
    if poly_rho and range_guard and kind == "asinh" and n <= 32:
        raise ValueError("range_guard is for exact radical evaluation")   # flash.py:835-836
    unit = 1.0 if kind == "softmax" else float(c)
    scale = 1.0 / (math.sqrt(D) * unit)
    has_sink = sink_logit is not None
    if has_sink:
        sink_in = np.asarray(sink_logit, np.float32).astype(F64)
        sink = np.broadcast_to(sink_in.reshape(-1), (H,)) / unit
        sink = cast(sink, "f32")
    else:
        sink = np.zeros(H)
    qs = cast(cast(q, "f32") * scale, dtype)                      # flash.py:833
    in_range = None
    if range_guard and kind == "asinh" and n <= 32:
        in_range = guard_in_range(qs, k, v, sink, var, has_sink)
        low, high = low_high(var)
        var = low if in_range else high
    o, o_res, stat = forward(qs, k, v, sink, var, has_sink, dtype, tiles)
    grads = None
    if do is not None:
        dq_s, dk, dv, dsink, _ = backward(qs, k, v, sink, o_res, stat, do, var, has_sink, dtype,
                                          tiles)
        dq = cast(cast(dq_s, "f32") * scale, dtype)               # VJP of flash.py:833
        if has_sink:
            d_in = dsink / unit                                    # VJP of flash.py:828
            if sink_in.size == H:
                d_logit = d_in.reshape(sink_in.shape)
            else:                                                  # one logit broadcast to H
                d_logit = np.full(sink_in.shape, d_in.sum())
            d_logit = cast(d_logit, "f32")
        else:
            d_logit = None
        grads = (dq, dk, dv, d_logit)
    return Result(o, stat, var, in_range, grads)


# ---------------------------------------------------------------------------
# dense references the reference's own tests compare against
# ---------------------------------------------------------------------------

def dense_asinh_attention(q, k, v, *, n, c, sink_logit=None, p_dtype="f64"):
    """algebraic.py:207-216 with asinh_power_weights :186-204, in float64.

    ``p_dtype`` rounds the weights before the PV product as the reference's
    ``p.astype(v.dtype)`` does (use "bf16" for bfloat16 values).
    """
    q, k, v = (np.asarray(a, F64) for a in (q, k, v))
    B, H, T, D = q.shape
    scores = _scores(q, k) * (1.0 / math.sqrt(D))
    mask = _causal(T)[None, None]
    x = scores / c
    m = np.max(np.where(mask, x, -1e30), axis=-1, keepdims=True)
    if sink_logit is not None:
        xb = np.broadcast_to(np.asarray(sink_logit, F64).reshape(1, -1, 1, 1), (1, H, 1, 1)) / c
        m = np.maximum(m, xb)
    shift = rho_exact(-m)[0]
    w = np.where(mask, ipow(rho_exact(x)[0] * shift, n), 0.0)
    denom = w.sum(-1, keepdims=True)
    if sink_logit is not None:
        denom = denom + ipow(rho_exact(xb)[0] * shift, n)
    p = w / denom
    return np.einsum("bhqk,bhkd->bhqd", cast(p, p_dtype), v)


def dense_softmax_attention(q, k, v, *, sink_logit=None, p_dtype="f64"):
    """standard.py:24-38 in float64."""
    q, k, v = (np.asarray(a, F64) for a in (q, k, v))
    B, H, T, D = q.shape
    s = _scores(q, k) * (1.0 / math.sqrt(D))
    mask = _causal(T)[None, None]
    s = np.where(mask, s, -1e30)
    if sink_logit is not None:
        bl = np.broadcast_to(np.asarray(sink_logit, F64).reshape(1, -1, 1, 1), (B, H, T, 1))
        full = np.concatenate([s, bl], -1)
    else:
        full = s
    full = full - full.max(-1, keepdims=True)
    e = np.exp(full)
    p = (e / e.sum(-1, keepdims=True))[..., :T]
    return np.einsum("bhqk,bhkd->bhqd", cast(p, p_dtype), v)
