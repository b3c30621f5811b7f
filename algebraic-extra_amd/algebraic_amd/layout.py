"""Layout moves of the model step as single-pass HIP kernels (libalgx.so).

``heads_to_tokens(a)``: the attention output (B, H, T, D) as (B, T, H * D),
``a.transpose(0, 2, 1, 3).reshape(B, T, d)`` of model.py:182, with rows of D
values moved whole; its gradient takes the inverse move.

``transpose_last2(x)``: (..., M, N) -> (..., N, M) contiguous, the
``swapaxes(X, -2, -1)`` of the Newton-Schulz iteration (optimizers.py:41,
:49, :58, :62): square blocks transposed in registers, or LDS tiles for
extents that are not multiples of 16 bytes.

``concat_cast(parts, dtype)``: float32 tensors (..., C_i) joined along the
last axis and cast to ``dtype`` (bf16 or float32) in one pass; the gradient
is split and cast back to float32 in one pass. The model's per-step
compute-dtype copies of the stacked weights for its fused projections.

``project(x, w)``: the model's projection ``x @ w`` (bf16, x (..., din), w
(din, dout)). Forward and input gradient are plain library GEMMs (hipBLASLt
through torch); the weight gradient ``x^T dY``, whose K is the batch's token
count while din x dout is one weight, runs on libalgx's split-K GEMM
(algx_gemm_bf16_splitk): the library's choice for these shapes leaves most
of the GPU idle (16 to 84 output tiles of 256 x 256 over 256 compute units).

The first two accept any dtype whose rows (heads_to_tokens: D elements) span a
multiple of 16 bytes (transpose_last2: 2- or 4-byte elements); all return new
contiguous tensors.
"""

import math

import ctypes

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


def _part_args(ts):
    arr = (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts])
    cols = (ctypes.c_int64 * len(ts))(*[t.shape[-1] for t in ts])
    return ctypes.cast(arr, ctypes.c_void_p), ctypes.cast(cols, ctypes.c_void_p), arr, cols


class _ConcatCast(torch.autograd.Function):
    @staticmethod
    def forward(ctx, dtype, *parts):
        parts = [_contig16(p) for p in parts]
        lead = parts[0].shape[:-1]
        rows = parts[0].numel() // parts[0].shape[-1]
        out = torch.empty(lead + (sum(p.shape[-1] for p in parts),), dtype=dtype,
                          device=parts[0].device)
        pp, cc, keep_a, keep_c = _part_args(parts)
        _lib.call("algx_concat_cast", pp, cc, len(parts), _lib.ptr(out), rows,
                  _lib.dtype_code(dtype), _lib.stream())
        ctx.shapes = [p.shape for p in parts]
        return out

    @staticmethod
    def backward(ctx, g):
        g = _contig16(g)
        grads = [torch.empty(sh, dtype=torch.float32, device=g.device) for sh in ctx.shapes]
        rows = grads[0].numel() // grads[0].shape[-1]
        pp, cc, keep_a, keep_c = _part_args(grads)
        _lib.call("algx_split_cast", _lib.ptr(g), pp, cc, len(grads), rows,
                  _lib.dtype_code(g.dtype), _lib.stream())
        return (None, *grads)


def concat_cast(parts, dtype: torch.dtype) -> torch.Tensor:
    """torch.cat(parts, -1).to(dtype) for float32 parts of one leading shape
    (last extents multiples of 4, at most 4 parts), as one pass each way."""
    parts = list(parts)
    if not 1 <= len(parts) <= 4:
        raise ValueError("concat_cast joins 1 to 4 parts")
    if any(p.dtype != torch.float32 for p in parts) or dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("concat_cast: float32 parts, bf16 or float32 output")
    if any(p.shape[:-1] != parts[0].shape[:-1] or p.shape[-1] % 4 for p in parts):
        raise ValueError("concat_cast: one leading shape, last extents multiples of 4")
    return _ConcatCast.apply(dtype, *parts)


__all__ = ["heads_to_tokens", "transpose_last2", "concat_cast"]


def splitk_splits(M: int, N: int, K: int) -> int:
    """Chunks of K for algx_gemm_bf16_splitk: the fewest (a power of two)
    whose workgroups cover 160 of the 256 compute units, keeping chunks of
    at least 256 rows that are whole 32-row stages."""
    tiles = math.ceil(M / 256) * math.ceil(N / 256)
    s = 1
    while tiles * s < 160 and K % (64 * s) == 0 and K // (2 * s) >= 256:
        s *= 2
    return s


def weight_grad(x2: torch.Tensor, g2: torch.Tensor) -> torch.Tensor:
    """x2^T g2 in bf16 for x2 (T, din), g2 (T, dout) bf16: float32 sums of
    split-K chunks added in chunk order (algx_gemm_bf16_splitk)."""
    T, din = x2.shape
    dout = g2.shape[1]
    x2, g2 = _contig16(x2), _contig16(g2)
    splits = splitk_splits(din, dout, T)
    ws = torch.empty(_lib.query("algx_gemm_bf16_splitk_workspace_bytes", din, dout, splits),
                     dtype=torch.uint8, device=x2.device)
    out = torch.empty((din, dout), dtype=torch.bfloat16, device=x2.device)
    _lib.call("algx_gemm_bf16_splitk", _lib.ptr(x2), _lib.ptr(g2), _lib.ptr(out), _lib.ptr(ws),
              din, dout, T, 0, 0, din, dout, dout, splits, _lib.stream())
    return out


class _Project(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w):
        ctx.save_for_backward(x, w)
        return x @ w

    @staticmethod
    def backward(ctx, g):
        x, w = ctx.saved_tensors
        din, dout = w.shape
        g = g.contiguous()
        dx = g @ w.t() if ctx.needs_input_grad[0] else None
        dw = None
        if ctx.needs_input_grad[1]:
            dw = weight_grad(x.reshape(-1, din), g.reshape(-1, dout))
        return dx, dw


def project(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x @ w with the weight gradient on the split-K GEMM (bf16, sizes whole
    multiples of 8 and a token count of whole 32-row stages); other inputs
    take torch's product and its autodiff."""
    din, dout = w.shape
    T = x.numel() // din if din else 0
    if (x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or not x.is_cuda
            or din % 8 or dout % 8 or T % 32 or T == 0):
        return x @ w
    return _Project.apply(x, w)

