"""QK RMS normalisation with a learned gain on MI355X.

Counterpart of ``algebraic.kernels.qk_norm`` (src/algebraic/kernels/qk_norm.py):
``qk_rms_norm(x, gain, eps=1e-5, *, block=1024)`` with the same validation,
computing ``rms_norm`` (algebraic.py:76-83) forward and its VJP with single-pass
HBM-bound HIP kernels. ``block`` is validated as in the reference (a row
count multiple aligned to 8) and otherwise only documents the caller's tiling.

``qk_rms_norm_pair(q, k, gain_q, gain_k)`` normalises the attention's q and k
in one launch each way; it returns exactly what two ``qk_rms_norm`` calls
return.
"""

import torch

from .. import _lib


class _NormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, gain, eps):
        rows = x.numel() // 64
        y = torch.empty_like(x)
        _lib.call("algx_qknorm_fwd", _lib.ptr(x), _lib.ptr(gain), _lib.ptr(y), rows, 64,
                  _lib.dtype_code(x.dtype), float(eps), _lib.stream())
        ctx.eps = eps
        ctx.save_for_backward(x, gain)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, gain = ctx.saved_tensors
        rows = x.numel() // 64
        dt = _lib.dtype_code(x.dtype)
        dy = dy.to(x.dtype).contiguous()
        dx = torch.empty_like(x)
        dgain = torch.empty(64, dtype=torch.float32, device=x.device)
        ws = torch.empty(max(1, _lib.query("algx_qknorm_bwd_workspace_bytes", rows, 64, dt)),
                         dtype=torch.uint8, device=x.device)
        _lib.call("algx_qknorm_bwd", _lib.ptr(x), _lib.ptr(gain), _lib.ptr(dy), _lib.ptr(dx),
                  _lib.ptr(dgain), _lib.ptr(ws), rows, 64, dt, float(ctx.eps), _lib.stream())
        return dx, dgain.to(gain.dtype), None


class _PairFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, gain_q, gain_k, eps):
        rows = q.numel() // 64
        yq, yk = torch.empty_like(q), torch.empty_like(k)
        _lib.call("algx_qknorm_pair_fwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(gain_q),
                  _lib.ptr(gain_k), _lib.ptr(yq), _lib.ptr(yk), rows, 64,
                  _lib.dtype_code(q.dtype), float(eps), _lib.stream())
        ctx.eps = eps
        ctx.save_for_backward(q, k, gain_q, gain_k)
        return yq, yk

    @staticmethod
    def backward(ctx, dyq, dyk):
        q, k, gain_q, gain_k = ctx.saved_tensors
        rows = q.numel() // 64
        dt = _lib.dtype_code(q.dtype)
        dyq = (torch.zeros_like(q) if dyq is None else dyq).to(q.dtype).contiguous()
        dyk = (torch.zeros_like(k) if dyk is None else dyk).to(k.dtype).contiguous()
        dxq, dxk = torch.empty_like(q), torch.empty_like(k)
        dgq = torch.empty(64, dtype=torch.float32, device=q.device)
        dgk = torch.empty(64, dtype=torch.float32, device=q.device)
        ws = torch.empty(max(1, _lib.query("algx_qknorm_pair_bwd_workspace_bytes", rows, 64, dt)),
                         dtype=torch.uint8, device=q.device)
        _lib.call("algx_qknorm_pair_bwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(gain_q),
                  _lib.ptr(gain_k), _lib.ptr(dyq), _lib.ptr(dyk), _lib.ptr(dxq), _lib.ptr(dxk),
                  _lib.ptr(dgq), _lib.ptr(dgk), _lib.ptr(ws), rows, 64, dt, float(ctx.eps),
                  _lib.stream())
        return dxq, dxk, dgq.to(gain_q.dtype), dgk.to(gain_k.dtype), None


def _check(x, gain, eps, block):
    if x.ndim < 2 or x.shape[-1] != 64 or tuple(gain.shape) != (64,):
        raise ValueError("QK RMS kernel needs D=64 and a one-dimensional gain")
    if x.dtype not in (torch.bfloat16, torch.float32) or gain.dtype != torch.float32:
        raise ValueError("QK RMS kernel needs float32/BF16 input and float32 gain")
    if block < 8 or block % 8 or x.numel() // 64 % block:
        raise ValueError("QK RMS row count must be divisible by a block aligned to eight rows")
    if eps <= 0:
        raise ValueError("QK RMS epsilon must be positive")


def qk_rms_norm(x, gain, eps=1e-5, *, block=1024):
    """RMS-normalize D=64 rows with a learned float32 gain (qk_norm.py:62-76)."""
    _check(x, gain, eps, block)
    return _NormFn.apply(x.contiguous(), gain.contiguous(), float(eps))


def qk_rms_norm_pair(q, k, gain_q, gain_k, eps=1e-5, *, block=1024):
    """``(qk_rms_norm(q, gain_q), qk_rms_norm(k, gain_k))`` in one launch each way.

    q and k must have the same shape and dtype (the attention's query and key
    tensors); each is validated as ``qk_rms_norm`` validates its input."""
    _check(q, gain_q, eps, block)
    _check(k, gain_k, eps, block)
    if q.shape != k.shape or q.dtype != k.dtype:
        raise ValueError("QK RMS pair needs q and k of one shape and dtype")
    return _PairFn.apply(q.contiguous(), k.contiguous(), gain_q.contiguous(),
                         gain_k.contiguous(), float(eps))
