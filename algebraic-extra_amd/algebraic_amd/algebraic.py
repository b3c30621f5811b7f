"""The model's elementwise algebraic ops on MI355X.

Counterparts of ``algebraic.algebraic.rms_norm`` and ``alu``
(src/algebraic/algebraic.py:76-117) for PyTorch-ROCm tensors, plus
``alu_glu(gate, up, beta)``: the feed-forward product ``gate * alu(up, beta)``
of model.py:186-191 in one pass, rounded as the two unfused bf16 ops round.
Forward and backward run as single-pass HBM-bound HIP kernels of libalgx.so
(include/algx.h); the backward of ``alu`` is the reference's custom VJP,
recomputing ``u`` and ``r`` from the saved input instead of storing them.

Inputs are bfloat16 or float32 CUDA (ROCm) tensors; ``rms_norm`` normalises
the last axis (a multiple of 8 values for bfloat16, of 4 for float32, at most
2048) and takes its gain as float32 (any other gain dtype is converted, and
its gradient returned in that dtype).
"""

from typing import Optional

import torch

from . import _lib


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """Contiguous with a 16-byte aligned base (the kernels move 16-byte vectors)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


class _RMSNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, gain, eps):
        D = x.shape[-1]
        rows = x.numel() // D if D else 0
        y = torch.empty_like(x)
        _lib.call("algx_rms_norm_fwd", _lib.ptr(x), _lib.ptr(gain), _lib.ptr(y), rows, D,
                  _lib.dtype_code(x.dtype), float(eps), _lib.stream())
        ctx.eps = eps
        ctx.save_for_backward(x, gain)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, gain = ctx.saved_tensors
        D = x.shape[-1]
        rows = x.numel() // D if D else 0
        dt = _lib.dtype_code(x.dtype)
        dy = _aligned(dy.to(x.dtype))
        dx = torch.empty_like(x)
        dgain = ws = None
        if gain is not None:
            dgain = torch.empty(D, dtype=torch.float32, device=x.device)
            ws = torch.empty(max(1, _lib.query("algx_rms_norm_bwd_workspace_bytes", rows, D, dt)),
                             dtype=torch.uint8, device=x.device)
        _lib.call("algx_rms_norm_bwd", _lib.ptr(x), _lib.ptr(gain), _lib.ptr(dy), _lib.ptr(dx),
                  _lib.ptr(dgain), _lib.ptr(ws), rows, D, dt, float(ctx.eps), _lib.stream())
        return dx, dgain, None


def rms_norm(x: torch.Tensor, gain: Optional[torch.Tensor], eps: float = 1e-5) -> torch.Tensor:
    """RMS normalization; ``gain=None`` gives the parameter-free AVN (algebraic.py:76-83)."""
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("rms_norm kernel needs float32 or bfloat16 input")
    D = x.shape[-1] if x.ndim else 0
    width = 8 if x.dtype == torch.bfloat16 else 4
    if D <= 0 or D % width or D > 2048:
        raise NotImplementedError(f"rms_norm kernel needs a last axis that is a multiple of {width}"
                                  f" and at most 2048, got {D}")
    if gain is not None and tuple(gain.shape) != (D,):
        raise ValueError(f"gain must have shape ({D},)")
    if not eps > 0:
        raise ValueError("rms_norm epsilon must be positive")
    if gain is None:
        return _RMSNormFn.apply(_aligned(x), None, float(eps))
    g32 = gain.to(torch.float32).contiguous()
    return _RMSNormFn.apply(_aligned(x), g32, float(eps))


class _AddRMSNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, r, gain, eps):
        D = x.shape[-1]
        rows = x.numel() // D if D else 0
        xsum, y = torch.empty_like(x), torch.empty_like(x)
        _lib.call("algx_add_rms_norm_fwd", _lib.ptr(x), _lib.ptr(r), _lib.ptr(gain),
                  _lib.ptr(xsum), _lib.ptr(y), rows, D, _lib.dtype_code(x.dtype), float(eps),
                  _lib.stream())
        ctx.eps = eps
        ctx.save_for_backward(xsum, gain)
        return xsum, y

    @staticmethod
    def backward(ctx, dxsum, dy):
        xsum, gain = ctx.saved_tensors
        D = xsum.shape[-1]
        rows = xsum.numel() // D if D else 0
        dt = _lib.dtype_code(xsum.dtype)
        dy = torch.zeros_like(xsum) if dy is None else _aligned(dy.to(xsum.dtype))
        dres = torch.zeros_like(xsum) if dxsum is None else _aligned(dxsum.to(xsum.dtype))
        dx = torch.empty_like(xsum)
        dgain = ws = None
        if gain is not None:
            dgain = torch.empty(D, dtype=torch.float32, device=xsum.device)
            ws = torch.empty(max(1, _lib.query("algx_rms_norm_bwd_workspace_bytes", rows, D, dt)),
                             dtype=torch.uint8, device=xsum.device)
        _lib.call("algx_add_rms_norm_bwd", _lib.ptr(xsum), _lib.ptr(gain), _lib.ptr(dy),
                  _lib.ptr(dres), _lib.ptr(dx), _lib.ptr(dgain), _lib.ptr(ws), rows, D, dt,
                  float(ctx.eps), _lib.stream())
        return dx, dx, dgain, None


def add_rms_norm(x: torch.Tensor, r: torch.Tensor, gain: Optional[torch.Tensor],
                 eps: float = 1e-5):
    """``(s, rms_norm(s, gain))`` for the residual sum ``s = x + r`` in one
    pass (the block's residual add followed by the next norm, model.py:177-178,
    :191, :166), rounded as the unfused add and norm round."""
    if x.shape != r.shape or x.dtype != r.dtype:
        raise ValueError("add_rms_norm needs x and r of one shape and dtype")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("rms_norm kernel needs float32 or bfloat16 input")
    D = x.shape[-1] if x.ndim else 0
    width = 8 if x.dtype == torch.bfloat16 else 4
    if D <= 0 or D % width or D > 2048:
        raise NotImplementedError(f"rms_norm kernel needs a last axis that is a multiple of {width}"
                                  f" and at most 2048, got {D}")
    if gain is not None and tuple(gain.shape) != (D,):
        raise ValueError(f"gain must have shape ({D},)")
    if not eps > 0:
        raise ValueError("rms_norm epsilon must be positive")
    g32 = None if gain is None else gain.to(torch.float32).contiguous()
    return _AddRMSNormFn.apply(_aligned(x), _aligned(r), g32, float(eps))


class _ALUFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, beta):
        y = torch.empty_like(x)
        _lib.call("algx_alu_fwd", _lib.ptr(x), _lib.ptr(y), x.numel(), _lib.dtype_code(x.dtype),
                  float(beta), _lib.stream())
        ctx.beta = beta
        ctx.save_for_backward(x)
        return y

    @staticmethod
    def backward(ctx, g):
        (x,) = ctx.saved_tensors
        g = _aligned(g.to(x.dtype))
        dx = torch.empty_like(x)
        _lib.call("algx_alu_bwd", _lib.ptr(x), _lib.ptr(g), _lib.ptr(dx), x.numel(),
                  _lib.dtype_code(x.dtype), float(ctx.beta), _lib.stream())
        return dx, None


def _check_float(*ts):
    dt = ts[0].dtype
    if dt not in (torch.bfloat16, torch.float32) or any(t.dtype != dt for t in ts):
        raise ValueError("alu kernels need float32 or bfloat16 tensors of one dtype")


def alu(x: torch.Tensor, beta: float = 1.0) -> torch.Tensor:
    """Algebraic linear unit ``x/2 (1 + bx / sqrt(1 + b^2 x^2))`` (algebraic.py:96-104)."""
    _check_float(x)
    return _ALUFn.apply(_aligned(x), float(beta))


class _ALUGLUFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gate, up, beta):
        out = torch.empty_like(up)
        _lib.call("algx_alu_glu_fwd", _lib.ptr(gate), _lib.ptr(up), _lib.ptr(out), up.numel(),
                  _lib.dtype_code(up.dtype), float(beta), _lib.stream())
        ctx.beta = beta
        ctx.save_for_backward(gate, up)
        return out

    @staticmethod
    def backward(ctx, dout):
        gate, up = ctx.saved_tensors
        dout = _aligned(dout.to(up.dtype))
        dgate, dup = torch.empty_like(gate), torch.empty_like(up)
        _lib.call("algx_alu_glu_bwd", _lib.ptr(gate), _lib.ptr(up), _lib.ptr(dout),
                  _lib.ptr(dgate), _lib.ptr(dup), up.numel(), _lib.dtype_code(up.dtype),
                  float(ctx.beta), _lib.stream())
        return dgate, dup, None


def alu_glu(gate: torch.Tensor, up: torch.Tensor, beta: float = 1.0) -> torch.Tensor:
    """``gate * alu(up, beta)`` in one pass (model.py:186-191)."""
    _check_float(gate, up)
    if gate.shape != up.shape:
        raise ValueError("alu_glu needs gate and up of one shape")
    return _ALUGLUFn.apply(_aligned(gate), _aligned(up), float(beta))


class _GLUPackedFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gu, act, beta):
        cols = gu.shape[-1] // 2
        rows = gu.numel() // (2 * cols)
        y = torch.empty(gu.shape[:-1] + (cols,), dtype=gu.dtype, device=gu.device)
        code = _lib.GLU_ALU if act == "alu" else _lib.GLU_SILU
        _lib.call("algx_glu_packed_fwd", _lib.ptr(gu), _lib.ptr(y), rows, cols, code,
                  _lib.dtype_code(gu.dtype), float(beta), _lib.stream())
        ctx.cfg = (code, beta)
        ctx.save_for_backward(gu)
        return y

    @staticmethod
    def backward(ctx, dy):
        (gu,) = ctx.saved_tensors
        code, beta = ctx.cfg
        cols = gu.shape[-1] // 2
        rows = gu.numel() // (2 * cols)
        dy = _aligned(dy.to(gu.dtype))
        dgu = torch.empty_like(gu)
        _lib.call("algx_glu_packed_bwd", _lib.ptr(gu), _lib.ptr(dy), _lib.ptr(dgu), rows, cols,
                  code, _lib.dtype_code(gu.dtype), float(beta), _lib.stream())
        return dgu, None, None


def glu_packed(gu: torch.Tensor, act: str = "alu", beta: float = 1.0) -> torch.Tensor:
    """``gate * act(up)`` for ``gu = [gate | up]`` on the last axis (one GEMM
    against ``[w_g | w_u]``, model.py:184-191): ``act="alu"`` is
    ``alu(up, beta)``, ``act="silu"`` is SwiGLU's ``up * sigmoid(up)``
    (standard.py:12-13). The gradient comes back packed the same way."""
    _check_float(gu)
    if act not in ("alu", "silu"):
        raise ValueError(f"unknown activation {act!r}")
    if gu.shape[-1] % 2:
        raise ValueError("glu_packed needs an even last axis [gate | up]")
    width = 8 if gu.dtype == torch.bfloat16 else 4
    if (gu.shape[-1] // 2) % width:
        raise NotImplementedError(f"glu_packed needs gate/up widths that are a multiple of {width}")
    return _GLUPackedFn.apply(_aligned(gu), act, float(beta))
