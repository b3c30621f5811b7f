"""Layout moves of the model step as single-pass HIP kernels (libalgx.so).

``heads_to_tokens(a)``: the attention output (B, H, T, D) as (B, T, H * D),
``a.transpose(0, 2, 1, 3).reshape(B, T, d)`` of model.py:182, with rows of D
values moved whole; its gradient takes the inverse move.

``transpose_last2(x)``: (..., M, N) -> (..., N, M) contiguous, the
``swapaxes(X, -2, -1)`` of the Newton-Schulz iteration (optimizers.py:41,
:49, :58, :62), through LDS tiles.

Both accept any dtype whose rows (heads_to_tokens: D elements) span a multiple
of 16 bytes (transpose_last2: 2- or 4-byte elements) and return new
contiguous tensors.
"""

import torch

from . import _lib


def _contig16(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _swap(x: torch.Tensor, B: int, P: int, Q: int, row: int) -> torch.Tensor:
    """(B, P, Q, row) -> (B, Q, P, row) as a new tensor of x's dtype."""
    x = _contig16(x)
    out = torch.empty((B, Q, P, row), dtype=x.dtype, device=x.device)
    _lib.call("algx_swap_axes", _lib.ptr(x), _lib.ptr(out), B, P, Q, row * x.element_size(),
              _lib.stream())
    return out


class _HeadsToTokens(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a):
        B, H, T, D = a.shape
        ctx.shape = (B, H, T, D)
        return _swap(a, B, H, T, D).view(B, T, H * D)

    @staticmethod
    def backward(ctx, g):
        B, H, T, D = ctx.shape
        return _swap(g, B, T, H, D)


def heads_to_tokens(a: torch.Tensor) -> torch.Tensor:
    """(B, H, T, D) -> (B, T, H * D) (model.py:182)."""
    if a.dim() != 4:
        raise ValueError("heads_to_tokens expects (B, H, T, D)")
    if (a.shape[-1] * a.element_size()) % 16:
        raise ValueError("heads_to_tokens: a row of D values must span a multiple of 16 bytes")
    return _HeadsToTokens.apply(a)


def _transpose(x: torch.Tensor) -> torch.Tensor:
    M, N = x.shape[-2], x.shape[-1]
    K = x.numel() // (M * N) if M * N else 0
    x = x.contiguous()
    out = torch.empty(x.shape[:-2] + (N, M), dtype=x.dtype, device=x.device)
    _lib.call("algx_transpose", _lib.ptr(x), _lib.ptr(out), K, M, N, x.element_size(),
              _lib.stream())
    return out


class _TransposeLast2(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        return _transpose(x)

    @staticmethod
    def backward(ctx, g):
        return _transpose(g)


def transpose_last2(x: torch.Tensor) -> torch.Tensor:
    """x.transpose(-2, -1) materialised contiguously (2- or 4-byte elements)."""
    if x.dim() < 2:
        raise ValueError("transpose_last2 needs at least 2 dimensions")
    if x.element_size() not in (2, 4):
        raise ValueError("transpose_last2: elements of 2 or 4 bytes")
    return _TransposeLast2.apply(x)


__all__ = ["heads_to_tokens", "transpose_last2"]
