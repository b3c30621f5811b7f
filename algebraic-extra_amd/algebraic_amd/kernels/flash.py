"""Causal flash attention with softmax or asinh-power weights on MI355X.

Drop-in counterpart of ``algebraic.kernels.flash`` (src/algebraic/kernels/flash.py)
for PyTorch-ROCm tensors: the same ``flash_attention`` signature, keyword
arguments, validation errors and numerics, with the device work done by the
gfx950 HIP kernels of libalgx.so (include/algx.h).

* softmax: weight ``exp(s - m)``, saved statistic ``m + log l``.
* asinh: kernel-unit score ``x = q.k / (sqrt(d) c)``, weight ``rho(x)^n`` with
  ``rho(x) = x + sqrt(1 + x^2)``; ``shift=True`` accumulates with a running
  maximum and ``(rho(x) rho(-m))^n``; ``shift=False`` accumulates unshifted,
  clamping scores at ``clamp`` unless the range guard has bounded them.
* ``range_guard=True`` (asinh, n <= 32) checks the input norms and value
  bound on the device and runs the unclamped unshifted kernel when in range,
  the shifted exact-rho kernel otherwise (flash.py:834-856). The choice is
  made on the GPU; the host never waits for it.

The TPU schedule flags (block sizes, resident/diagonal/head-resident
backends, compact statistics) are validated exactly as the reference does but
select nothing here: one MFMA schedule serves every case. ``poly_rho`` (the
reference's opt-in bounded radical, radical.py:26-38) evaluates rho and its
slope by the reference's degree-4 polynomials where |x| <= 1 and exactly
elsewhere; the reference makes that choice once per Pallas score tile, the
kernels here per score (the two agree to ~3e-5 relative).
"""

import math
from typing import NamedTuple, Optional

import torch

from .. import _lib

LANES = 128
NEG = -1e4


class Variant(NamedTuple):
    """Static kernel configuration, field-for-field as flash.py:59-73."""
    kind: str
    n: int = 16
    shift: bool = True
    fast_rho: bool = False
    clamp: float = 0.0
    inv_stat: bool = False
    compact_stat: bool = False
    poly_rho: bool = False
    bounded_scores: bool = False
    resident_bwd: bool = False
    diagonal_bwd: bool = False
    diagonal_fwd: bool = False
    head_resident: bool = False
    precise_output: bool = False


def _root(value: float, n: int) -> float:
    """value^(1/n) for n a power of two, by repeated square roots (flash.py:117-123)."""
    out = float(value)
    while n > 1:
        out = math.sqrt(out)
        n //= 2
    return out


def make_variant(kind: str, n: int = 16, c: float = 16.0, seq_len: int = 2048,
                 shift: Optional[bool] = None, fast_rho: Optional[bool] = None,
                 inv_stat: Optional[bool] = None, compact_stat: bool = True,
                 poly_rho: bool = False) -> Variant:
    """Same rules and errors as flash.py:732-760."""
    if kind == "softmax":
        return Variant("softmax", compact_stat=bool(compact_stat))
    if kind != "asinh":
        raise ValueError(f"unknown attention kernel: {kind}")
    if n < 2 or n & (n - 1):
        raise ValueError("asinh kernel needs n to be a power of two")
    if not math.isfinite(c) or c <= 0:
        raise ValueError("asinh scale c must be positive and finite")
    # rho((t - 1/t)/2) = t with (T+1) t^n = 1e37 bounds the denominator.
    t = _root(1e37 / (seq_len + 1), n)
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


def _c_variant(var: Variant) -> _lib.AttnVariant:
    return _lib.AttnVariant(
        kind=_lib.SOFTMAX if var.kind == "softmax" else _lib.ASINH, n=int(var.n),
        shift=int(var.shift), fast_rho=int(var.fast_rho), inv_stat=int(var.inv_stat),
        bounded_scores=int(var.bounded_scores), precise_output=int(var.precise_output),
        clamp=float(var.clamp), poly_rho=int(var.poly_rho))


class _Plan(NamedTuple):
    low: Variant
    high: Optional[Variant]      # set when the range guard dispatches
    q_scale: float
    bound: float
    vmax: float
    has_sink: bool


class _FlashFn(torch.autograd.Function):
    """Custom VJP of flash.py:708-729 (residuals q, k, v, sink, o, stat)."""

    @staticmethod
    def forward(ctx, q, k, v, sink, plan: _Plan):
        B, H, T, D = q.shape
        dt = _lib.dtype_code(q.dtype)
        dev = q.device
        st = _lib.stream()
        guard = None
        if plan.high is not None:
            words = _lib.query("algx_attn_guard_words")
            guard = torch.empty(words, dtype=torch.int32, device=dev)
        # One call: q_s = cast(q * scale) (flash.py:833), the guard word when
        # guarded (:834-849) and the forward (:853-856).
        q_s = torch.empty_like(q)
        o = torch.empty_like(q)
        stat = torch.empty((B, H, T), dtype=torch.float32, device=dev)
        precise = plan.low.precise_output or (plan.high is not None and plan.high.precise_output)
        o_precise = torch.empty(q.shape, dtype=torch.float32, device=dev) if precise else None
        ws = None
        if guard is not None:
            ws = torch.empty(_lib.query("algx_attn_forward_workspace_bytes", B, H, T, D),
                             dtype=torch.uint8, device=dev)
        # When a backward will follow, its workspace is allocated here and
        # prepared by the forward in passing (its dQ accumulator cleared).
        bws = None
        if any(ctx.needs_input_grad[:4]):
            bws = torch.empty(_lib.query("algx_attn_bwd_workspace_bytes", B, H, T, D),
                              dtype=torch.uint8, device=dev)
        lo = _c_variant(plan.low)
        hi = _c_variant(plan.high) if plan.high is not None else None
        _lib.call("algx_attn_forward", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(sink),
                  _lib.ptr(q_s), _lib.ptr(o), _lib.ptr(o_precise), _lib.ptr(stat),
                  _lib.ptr(guard), _lib.ptr(ws), _lib.ptr(bws), B, H, T, D, dt, plan.q_scale,
                  plan.bound, plan.vmax, lo, hi, st)
        ctx.plan = plan
        ctx.bws = bws
        ctx.save_for_backward(q_s, k, v, sink, o, o_precise, stat, guard)
        return o

    @staticmethod
    def backward(ctx, do):
        q_s, k, v, sink, o, o_precise, stat, guard = ctx.saved_tensors
        plan = ctx.plan
        B, H, T, D = q_s.shape
        dt = _lib.dtype_code(q_s.dtype)
        do = do.to(q_s.dtype).contiguous()
        dq, dk, dv = torch.empty_like(q_s), torch.empty_like(k), torch.empty_like(v)
        dsink = torch.empty((H,), dtype=torch.float32, device=q_s.device) if sink is not None else None
        # The forward's prepared workspace serves one backward; a second one
        # (retain_graph) hands it over as raw memory.
        ws, state = ctx.bws, _lib.ATTN_WS_CLEARED
        ctx.bws = None
        if ws is None:
            ws = torch.empty(_lib.query("algx_attn_bwd_workspace_bytes", B, H, T, D),
                             dtype=torch.uint8, device=q_s.device)
            state = _lib.ATTN_WS_RAW
        lo = _c_variant(plan.low)
        hi = _c_variant(plan.high) if plan.high is not None else None
        _lib.call("algx_attn_bwd", _lib.ptr(q_s), _lib.ptr(k), _lib.ptr(v), _lib.ptr(sink),
                  _lib.ptr(o), _lib.ptr(o_precise), _lib.ptr(stat), _lib.ptr(do),
                  _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(dsink), _lib.ptr(ws), state,
                  B, H, T, D, dt, plan.q_scale, lo, hi, _lib.ptr(guard), _lib.stream())
        return dq, dk, dv, dsink, None


def flash_attention(q, k, v, sink_logit: Optional[torch.Tensor] = None, *, kind: str = "softmax",
                    n: int = 16, c: float = 16.0, block: int = 512,
                    block_q: Optional[int] = None, block_k: Optional[int] = None,
                    shift: Optional[bool] = None, fast_rho: Optional[bool] = None,
                    inv_stat: Optional[bool] = None, compact_stat: bool = True,
                    poly_rho: bool = False, range_guard: bool = False,
                    resident_bwd: Optional[bool] = None,
                    diagonal_bwd: Optional[bool] = None,
                    diagonal_fwd: Optional[bool] = None,
                    head_resident: Optional[bool] = None):
    """Causal attention on (B, H, T, D); ``sink_logit`` broadcastable to (H,).

    Signature, defaults and ValueErrors of flash.py:763-857. Inputs are
    bfloat16 or float32 CUDA (ROCm) tensors of one dtype; the output has q's
    dtype. Differentiable in q, k, v and sink_logit.
    """
    B, H, T, D = q.shape
    bq = min(block_q or block, T)
    bk = min(block_k or block, T)
    if T % bq or T % bk:
        raise ValueError(f"sequence length {T} must be divisible by blocks ({bq}, {bk})")
    var = make_variant(kind, n, c, T, shift, fast_rho, inv_stat, compact_stat, poly_rho)
    bf16 = q.dtype == k.dtype == v.dtype == torch.bfloat16
    resident_supported = (T in (512, 1024, 2048) and D == 64 and bf16 and not poly_rho and
                          (kind == "softmax" or n == 16))
    if resident_bwd is True and not resident_supported:
        raise ValueError("resident backward needs bfloat16, T=512/1024/2048, D=64, "
                         "and softmax or exact asinh n=16")
    use_resident = (resident_supported and T == 2048 and bq == bk == 512 and compact_stat
                    if resident_bwd is None else bool(resident_bwd))
    if diagonal_bwd is True and not use_resident:
        raise ValueError("diagonal backward requires the resident backward backend")
    head_supported = use_resident and T == 2048 and bq == bk == 512 and compact_stat
    if head_resident is True and not head_supported:
        raise ValueError("whole-head residency needs resident bfloat16 T=2048,D=64, "
                         "512-square public tiles, and compact statistics")
    if q.dtype not in (torch.bfloat16, torch.float32) or not (q.dtype == k.dtype == v.dtype):
        raise ValueError("flash_attention needs q, k, v of one dtype, bfloat16 or float32")
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k and v must share the shape (B, H, T, D)")
    if D not in (16, 32, 64):
        raise ValueError(f"head dimension {D} is not supported (16, 32 or 64)")
    unit = 1.0 if kind == "softmax" else float(c)
    scale = 1.0 / (math.sqrt(D) * unit)
    has_sink = sink_logit is not None
    if has_sink:
        sink_in = torch.as_tensor(sink_logit, device=q.device).to(torch.float32)
        sink = (torch.broadcast_to(sink_in.reshape(-1), (H,)) / unit).contiguous()
    else:
        sink = None
    if range_guard and kind == "asinh" and n <= 32:
        if poly_rho:
            raise ValueError("range_guard is for exact radical evaluation")  # flash.py:835-836
        bound = min(16.0, var.clamp / 2)
        vmax = min(1e8, 1e37 / ((T + int(has_sink)) * (2 * bound + 1) ** n))
        low = var._replace(shift=False, inv_stat=True, bounded_scores=True)
        high = var._replace(shift=True, inv_stat=False, fast_rho=False, bounded_scores=False,
                            head_resident=False, precise_output=True)
        plan = _Plan(low, high, scale, bound, vmax, has_sink)
    else:
        plan = _Plan(var, None, scale, 0.0, 0.0, has_sink)
    return _FlashFn.apply(q.contiguous(), k.contiguous(), v.contiguous(), sink, plan)
