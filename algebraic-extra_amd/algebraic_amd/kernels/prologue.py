"""Attention prologue of the model block on MI355X: projections -> attention inputs.

The reference's block (src/algebraic/model.py:166-174) reshapes the q, k, v
projections to (B, H, T, D), RMS-normalises q and k over D with learned gains
(qk_norm), and rotates them with the position tables (apply_rotary,
algebraic.py:172-179). ``attention_prologue`` does all of it, with the
layout change, in one HIP pass that reads the (B, T, 3 d) output of a fused
QKV projection in place; its backward writes the gradient of that buffer in
one pass. Results are those of the unfused operators, rounding included.
"""

from typing import Optional

import torch

from .. import _lib


class _PrologueFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, qkv, q_gain, k_gain, cos, sin, H, eps):
        B, T, three_d = qkv.shape
        d = three_d // 3
        D = d // H
        dt = _lib.dtype_code(qkv.dtype)
        out = torch.empty((3, B, H, T, D), dtype=qkv.dtype, device=qkv.device)
        base = qkv.data_ptr()
        esz = qkv.element_size()
        _lib.call("algx_qk_prologue_fwd", _lib.c_ptr(base), _lib.c_ptr(base + d * esz),
                  _lib.c_ptr(base + 2 * d * esz), three_d, _lib.ptr(q_gain), _lib.ptr(k_gain),
                  _lib.ptr(cos), _lib.ptr(sin), _lib.ptr(out[0]), _lib.ptr(out[1]),
                  _lib.ptr(out[2]), B, T, H, D, dt, float(eps), _lib.stream())
        ctx.H, ctx.eps = H, eps
        ctx.save_for_backward(qkv, q_gain, k_gain, cos, sin)
        return out[0], out[1], out[2]

    @staticmethod
    def backward(ctx, dq_out, dk_out, dv_out):
        qkv, q_gain, k_gain, cos, sin = ctx.saved_tensors
        B, T, three_d = qkv.shape
        d = three_d // 3
        H = ctx.H
        D = d // H
        dt = _lib.dtype_code(qkv.dtype)
        grads = [torch.zeros((B, H, T, D), dtype=qkv.dtype, device=qkv.device) if g is None
                 else g.to(qkv.dtype).contiguous() for g in (dq_out, dk_out, dv_out)]
        dqkv = torch.empty_like(qkv)
        dqg = dkg = ws = None
        if q_gain is not None:
            dqg = torch.empty(D, dtype=torch.float32, device=qkv.device)
            dkg = torch.empty(D, dtype=torch.float32, device=qkv.device)
            ws = torch.empty(max(1, _lib.query("algx_qk_prologue_bwd_workspace_bytes", B, T, H, D,
                                               dt)), dtype=torch.uint8, device=qkv.device)
        base = dqkv.data_ptr()
        esz = dqkv.element_size()
        qb = qkv.data_ptr()
        _lib.call("algx_qk_prologue_bwd", _lib.c_ptr(qb), _lib.c_ptr(qb + d * esz),
                  _lib.ptr(q_gain), _lib.ptr(k_gain), _lib.ptr(cos), _lib.ptr(sin),
                  _lib.ptr(grads[0]), _lib.ptr(grads[1]), _lib.ptr(grads[2]), _lib.c_ptr(base),
                  _lib.c_ptr(base + d * esz), _lib.c_ptr(base + 2 * d * esz), three_d,
                  _lib.ptr(dqg), _lib.ptr(dkg), _lib.ptr(ws), B, T, H, D, dt, float(ctx.eps),
                  _lib.stream())
        return dqkv, dqg, dkg, None, None, None, None


def attention_prologue(qkv: torch.Tensor, n_heads: int, q_gain: Optional[torch.Tensor],
                       k_gain: Optional[torch.Tensor], cos: Optional[torch.Tensor],
                       sin: Optional[torch.Tensor], eps: float = 1e-5):
    """(q, k, v) in (B, H, T, 64) from a (B, T, 3 H 64) projection output.

    q and k are RMS-normalised over the head dimension with the float32 gains
    (both None: no norm) and rotated by the (T, 32) float32 tables (both
    None: no rotation)."""
    if qkv.ndim != 3 or qkv.shape[-1] % 3 or (qkv.shape[-1] // 3) != n_heads * 64:
        raise ValueError("attention_prologue needs a (B, T, 3 * n_heads * 64) projection")
    if qkv.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("attention_prologue needs bfloat16 or float32 projections")
    if (q_gain is None) != (k_gain is None) or (cos is None) != (sin is None):
        raise ValueError("gains and tables come in pairs")
    T = qkv.shape[1]
    g32 = [None if g is None else g.to(torch.float32).contiguous() for g in (q_gain, k_gain)]
    tabs = [None if t is None else t[:T].to(torch.float32).contiguous() for t in (cos, sin)]
    if tabs[0] is not None and tuple(tabs[0].shape) != (T, 32):
        raise ValueError("rotation tables must be (T, 32)")
    return _PrologueFn.apply(qkv.contiguous(), g32[0], g32[1], tabs[0], tabs[1], int(n_heads),
                             float(eps))
