"""QK RMS normalisation with a learned gain on MI355X.

Counterpart of ``algebraic.kernels.qk_norm`` (src/algebraic/kernels/qk_norm.py):
``qk_rms_norm(x, gain, eps=1e-5, *, block=1024)`` with the same validation,
computing ``rms_norm`` (algebraic.py:76-83) forward and its VJP with single-pass
HBM-bound HIP kernels. ``block`` is validated as in the reference (a row
count multiple aligned to 8) and otherwise only documents the caller's tiling.
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


def qk_rms_norm(x, gain, eps=1e-5, *, block=1024):
    """RMS-normalize D=64 rows with a learned float32 gain (qk_norm.py:62-76)."""
    if x.ndim < 2 or x.shape[-1] != 64 or tuple(gain.shape) != (64,):
        raise ValueError("QK RMS kernel needs D=64 and a one-dimensional gain")
    if x.dtype not in (torch.bfloat16, torch.float32) or gain.dtype != torch.float32:
        raise ValueError("QK RMS kernel needs float32/BF16 input and float32 gain")
    if block < 8 or block % 8 or x.numel() // 64 % block:
        raise ValueError("QK RMS row count must be divisible by a block aligned to eight rows")
    if eps <= 0:
        raise ValueError("QK RMS epsilon must be positive")
    return _NormFn.apply(x.contiguous(), gain.contiguous(), float(eps))
