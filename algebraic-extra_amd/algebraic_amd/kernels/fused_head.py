"""Fused tied-embedding projection and likelihood loss on MI355X.

Counterpart of ``algebraic.kernels.fused_head`` (src/algebraic/kernels/fused_head.py):
``fused_head(h, embed, targets, *, kind="ce", n=16, c=16.0, block_n=128,
block_v=512)`` returns ``(objective, telemetry)`` exactly as the reference:

* ``ce``: mean cross-entropy and the per-token NLL ``lse - z_t``;
* ``alg_ce``: likelihood ``p_j ~ rho(z_j/c)^n`` with the argument clamped at
  ``0.25 (1e38/V)^(1/n)``; the objective is ``mean(1 - p_t)`` and its VJP is
  the exact log-likelihood gradient ``(n/c) r_j (p_j - y_j) / N``; the
  telemetry is the target probability.

The (N, V) logits are never materialised: the HIP kernels stream vocabulary
tiles through LDS with bf16 MFMA and keep per-token statistics in registers.
``block_n`` is validated as in the reference (N must be divisible by it);
``block_v`` only documents the caller's tiling.
"""

import math

import torch

from .. import _lib


def _root(value, n):
    out = float(value)
    while n > 1:
        out = math.sqrt(out)
        n //= 2
    return out


def _ipow(x, n):
    out, base = None, x
    while n:
        if n & 1:
            out = base if out is None else out * base
        n >>= 1
        if n:
            base = base * base
    return out


def _telemetry(stat, zt, kind, n, c, clamp):
    """(per-token NLL or target probability, objective), fused_head.py:219-229."""
    if kind == "ce":
        nll = stat - zt
        return nll, nll.mean()
    x = torch.clamp(zt / c, max=clamp)
    rad = 1.0 + x * x
    t = x.abs() + rad * torch.rsqrt(rad)
    rho = torch.where(x >= 0, t, 1.0 / t)
    pt = _ipow(rho * stat, n)
    return pt, (1.0 - pt).mean()


class _HeadFn(torch.autograd.Function):
    """Custom VJP of fused_head.py:232-257 (residuals h, E, targets, stat)."""

    @staticmethod
    def forward(ctx, h, embed, targets, kind, n, c, clamp):
        N, d = h.shape
        V = embed.shape[0]
        e = embed.to(h.dtype).contiguous()                    # fused_head.py:168
        stat = torch.empty(N, dtype=torch.float32, device=h.device)
        zt = torch.empty(N, dtype=torch.float32, device=h.device)
        kcode = _lib.HEAD_CE if kind == "ce" else _lib.HEAD_ALG_CE
        dt = _lib.dtype_code(h.dtype)
        ws = torch.empty(max(1, _lib.query("algx_head_fwd_workspace_bytes", N, d, V, dt)),
                         dtype=torch.uint8, device=h.device)
        _lib.call("algx_head_fwd", _lib.ptr(h), _lib.ptr(e), _lib.ptr(targets), _lib.ptr(stat),
                  _lib.ptr(zt), _lib.ptr(ws), N, d, V, kcode, int(n), float(1.0 / c),
                  float(clamp), dt, _lib.stream())
        tel, obj = _telemetry(stat, zt, kind, n, c, clamp)
        ctx.cfg = (kind, n, c, clamp, embed.dtype)
        ctx.save_for_backward(h, e, targets, stat)
        ctx.mark_non_differentiable(tel)
        return obj, tel

    @staticmethod
    def backward(ctx, g_obj, g_tel):
        h, e, targets, stat = ctx.saved_tensors
        kind, n, c, clamp, embed_dtype = ctx.cfg
        N, d = h.shape
        V = e.shape[0]
        dt = _lib.dtype_code(h.dtype)
        slope = 1.0 if kind == "ce" else n / c
        scale = (g_obj.to(torch.float32) * (slope / N)).reshape(1).contiguous()
        dh = torch.empty_like(h)
        de = torch.empty((V, d), dtype=torch.float32, device=h.device)
        ws = torch.empty(max(1, _lib.query("algx_head_bwd_workspace_bytes", N, d, V, dt)),
                         dtype=torch.uint8, device=h.device)
        kcode = _lib.HEAD_CE if kind == "ce" else _lib.HEAD_ALG_CE
        _lib.call("algx_head_bwd", _lib.ptr(h), _lib.ptr(e), _lib.ptr(targets), _lib.ptr(stat),
                  _lib.ptr(scale), _lib.ptr(dh), _lib.ptr(de), _lib.ptr(ws), N, d, V, kcode,
                  int(n), float(1.0 / c), float(clamp), dt, _lib.stream())
        return dh, de.to(embed_dtype), None, None, None, None, None


def fused_head(h, embed, targets, *, kind="ce", n=16, c=16.0, block_n=128, block_v=512):
    """Fused tied-embedding projection and likelihood objective (fused_head.py:260-275).

    ``h`` (N, d) hidden states, ``embed`` (V, d), ``targets`` (N,). Returns
    ``(objective, telemetry)``; telemetry carries no gradient.
    """
    if kind not in ("ce", "alg_ce"):
        raise ValueError(kind)
    if kind == "alg_ce" and (n & (n - 1)):
        raise ValueError("n must be a power of two")
    N, d = h.shape
    bn = min(block_n, N)
    if N % bn:
        raise ValueError(f"token count {N} must be divisible by block {bn}")
    if h.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("fused_head needs bfloat16 or float32 hidden states")
    if embed.ndim != 2 or embed.shape[1] != d:
        raise ValueError("embed must be (V, d) with the hidden width d")
    clamp = 0.25 * _root(1e38 / embed.shape[0], n) if kind == "alg_ce" else 0.0
    t32 = targets.to(device=h.device, dtype=torch.int32).contiguous()
    obj, tel = _HeadFn.apply(h.contiguous(), embed, t32, kind, int(n), float(c), float(clamp))
    return obj, tel.detach()
