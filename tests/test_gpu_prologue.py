"""GPU parity of the fused attention prologue (QK-norm + rotation + layout).

Against the CPU oracle (tolerances of tests/_tol.py) and against the unfused
operators it replaces -- qk_rms_norm, the torch rotate-half product and the
(B, T, H, D) -> (B, H, T, D) transpose -- which, rounding to bf16 at the same
points, it must match bit for bit in outputs and input gradients.
"""

import numpy as np
import pytest
import torch

from _tol import assert_bf16, assert_f32, rel_l2, to_np
from algebraic_amd.kernels import qk_rms_norm
from algebraic_amd.kernels.prologue import attention_prologue
from algebraic_amd.model import apply_rotary, cayley_table_geometric, rope_table
from oracle import prologue as OP

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(B, T, H, dtype, seed, tables="cayley"):
    g = torch.Generator(device=DEV).manual_seed(seed)
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    qkv = (2 * torch.randn((B, T, 3 * H * 64), generator=g, device=DEV)).to(tdt)
    qg = 1 + 0.2 * torch.randn(64, generator=g, device=DEV)
    kg = 1 + 0.2 * torch.randn(64, generator=g, device=DEV)
    if tables == "cayley":
        cos, sin = cayley_table_geometric(64, T, device=DEV)
    else:
        cos, sin = rope_table(64, T, device=DEV)
    dout = [torch.randn((B, H, T, 64), generator=g, device=DEV).to(tdt) for _ in range(3)]
    return qkv, qg, kg, cos, sin, dout


def _unfused(qkv, H, qg, kg, cos, sin, eps):
    B, T, _ = qkv.shape
    q, k, v = qkv.view(B, T, 3, H, 64).unbind(2)
    q, k, v = (t.transpose(1, 2) for t in (q, k, v))
    if qg is not None:
        q, k = qk_rms_norm(q, qg, eps, block=8), qk_rms_norm(k, kg, eps, block=8)
    if cos is not None:
        q, k = apply_rotary(q, cos, sin), apply_rotary(k, cos, sin)
    return q, k, v.contiguous()


def _grads(fn, qkv, qg, kg, dout):
    x = qkv.clone().requires_grad_(True)
    gq = qg.clone().requires_grad_(True) if qg is not None else None
    gk = kg.clone().requires_grad_(True) if kg is not None else None
    outs = fn(x, gq, gk)
    torch.autograd.backward(outs, dout)
    torch.cuda.synchronize()
    return outs, x.grad, (gq.grad if gq is not None else None), (gk.grad if gk is not None else None)


@pytest.mark.parametrize("norm,rot", [(True, True), (False, True), (True, False)])
@pytest.mark.parametrize("B,T,H", [(2, 100, 3), (1, 600, 2)])
def test_prologue_equals_unfused_bf16(norm, rot, B, T, H):
    """Ragged T (100: not a multiple of a wave's rows; 600: a partial 512-token
    segment)."""
    qkv, qg, kg, cos, sin, dout = _inputs(B, T, H, "bf16", 7)
    qg, kg = (qg, kg) if norm else (None, None)
    cs = (cos, sin) if rot else (None, None)
    f = _grads(lambda x, a, b: attention_prologue(x, H, a, b, *cs), qkv, qg, kg, dout)
    u = _grads(lambda x, a, b: _unfused(x, H, a, b, *cs, 1e-5), qkv, qg, kg, dout)
    for a, b in zip(f[0], u[0]):
        assert a.is_contiguous() and torch.equal(a, b)
    assert torch.equal(f[1], u[1])
    if norm:
        assert rel_l2(f[2], u[2]) <= 1e-5 and rel_l2(f[3], u[3]) <= 1e-5


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("tables", ["cayley", "rope"])
def test_prologue_matches_oracle(dtype, tables):
    B, T, H = 2, 40, 2
    eps = 1e-5
    qkv, qg, kg, cos, sin, dout = _inputs(B, T, H, dtype, 11, tables)
    outs, dqkv, dqg, dkg = _grads(lambda x, a, b: attention_prologue(x, H, a, b, cos, sin, eps),
                                  qkv, qg, kg, dout)
    x = to_np(qkv).reshape(B, T, 3, H, 64)
    check = assert_f32 if dtype == "f32" else assert_bf16
    d = to_np(dqkv).reshape(B, T, 3, H, 64)
    for i, gain, dg in ((0, qg, dqg), (1, kg, dkg)):
        want = OP.forward(x[:, :, i], to_np(gain), to_np(cos), to_np(sin), eps, dtype)
        check(outs[i], want, what=f"out{i}")
        wdx, wdg = OP.backward(x[:, :, i], to_np(gain), to_np(cos), to_np(sin), to_np(dout[i]),
                               eps, dtype)
        check(d[:, :, i], wdx, what=f"dx{i}")
        assert rel_l2(dg, wdg) <= (1e-5 if dtype == "f32" else 1e-3)
    np.testing.assert_array_equal(to_np(outs[2]), np.transpose(x[:, :, 2], (0, 2, 1, 3)))
    np.testing.assert_array_equal(d[:, :, 2], np.transpose(to_np(dout[2]), (0, 2, 1, 3)))


def test_prologue_at_model_shape():
    """The 350M block's shape: B=8, T=2048, H=16, bf16, Cayley tables."""
    B, T, H = 8, 2048, 16
    qkv, qg, kg, cos, sin, dout = _inputs(B, T, H, "bf16", 13)
    f = _grads(lambda x, a, b: attention_prologue(x, H, a, b, cos, sin), qkv, qg, kg, dout)
    u = _grads(lambda x, a, b: _unfused(x, H, a, b, cos, sin, 1e-5), qkv, qg, kg, dout)
    for a, b in zip(f[0], u[0]):
        assert torch.equal(a, b)
    assert torch.equal(f[1], u[1])
    assert rel_l2(f[2], u[2]) <= 1e-5 and rel_l2(f[3], u[3]) <= 1e-5
