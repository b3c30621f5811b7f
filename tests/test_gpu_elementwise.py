"""GPU parity of rms_norm, alu and alu_glu (HIP) against the CPU oracle.

Same seeded inputs on both sides, tolerances of tests/_tol.py; the model's
shapes (d_model 768/1024 rows, the 350M feed-forward width 2688) at full size
on the GPU, checked against the oracle on a slice of rows and, for the
reductions over all rows (dgain), against a float64 reduction.
"""

import numpy as np
import pytest
import torch

from _tol import assert_bf16, assert_f32, rel_l2, to_np
from algebraic_amd.algebraic import alu, alu_glu, rms_norm
from oracle import elementwise as OE

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _tdt(dtype):
    return torch.float32 if dtype == "f32" else torch.bfloat16


def _check(dtype):
    return assert_f32 if dtype == "f32" else assert_bf16


def _randn(rng, shape, dtype, scale=1.0):
    return torch.from_numpy((scale * rng.standard_normal(shape)).astype(np.float32)).to(_tdt(dtype))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("with_gain", [False, True])
@pytest.mark.parametrize("rows,D", [(1, 8), (37, 64), (129, 776), (300, 768), (64, 1024),
                                    (5, 1016), (40, 1536), (9, 1288), (3, 2048)])
def test_rms_norm_output_and_vjp(dtype, with_gain, rows, D):
    """Ragged widths (776 = 97 bf16 chunks, 1016 = 254 f32 chunks, 1288 =
    322 f32 chunks) leave lanes idle in a row's last chunk; 1536 is the 1b
    preset's d_model and 2048 the widest row; row 0 is zero (tau = eps^-1/2,
    dx = tau dy)."""
    if D % (8 if dtype == "bf16" else 4):
        pytest.skip("width not a multiple of the vector")
    rng = np.random.default_rng(1000 + rows + D)
    eps = 1e-5
    x = _randn(rng, (rows, D), dtype, 3.0)
    x[0] = 0
    dy = _randn(rng, (rows, D), dtype)
    gain = torch.from_numpy((1 + 0.1 * rng.standard_normal(D)).astype(np.float32)) if with_gain else None
    tx = x.to(DEV).requires_grad_(True)
    tg = gain.to(DEV).requires_grad_(True) if with_gain else None
    y = rms_norm(tx, tg, eps)
    y.backward(dy.to(DEV))
    torch.cuda.synchronize()
    g_np = to_np(gain) if with_gain else None
    _check(dtype)(y, OE.rms_norm(to_np(x), g_np, eps, dtype), what="y")
    want_dx, want_dg = OE.rms_norm_vjp(to_np(x), g_np, to_np(dy), eps, dtype)
    _check(dtype)(tx.grad, want_dx, what="dx")
    if with_gain:
        assert tg.grad.dtype == torch.float32
        assert rel_l2(tg.grad, want_dg) <= (1e-5 if dtype == "f32" else 1e-3)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("D", [768, 1024])
def test_rms_norm_at_model_shape(dtype, D):
    """16384 rows (8 x 2048 tokens) of d_model values with a gain, as ln1/ln2."""
    rows = 16384
    rng = np.random.default_rng(D)
    eps = 1e-5
    x = _randn(rng, (8, 2048, D), dtype, 2.0)
    dy = _randn(rng, (8, 2048, D), dtype)
    gain = torch.from_numpy((1 + 0.1 * rng.standard_normal(D)).astype(np.float32))
    tx = x.to(DEV).requires_grad_(True)
    tg = gain.to(DEV).requires_grad_(True)
    y = rms_norm(tx, tg, eps)
    y.backward(dy.to(DEV))
    torch.cuda.synchronize()
    sl = (slice(0, 1), slice(0, 512))
    _check(dtype)(y[sl], OE.rms_norm(to_np(x[sl]), to_np(gain), eps, dtype), what="y")
    want_dx, _ = OE.rms_norm_vjp(to_np(x[sl]), to_np(gain), to_np(dy[sl]), eps, dtype)
    _check(dtype)(tx.grad[sl], want_dx, what="dx")
    xf = x.to(DEV).double().reshape(rows, D)
    tau = torch.rsqrt((xf * xf).mean(-1, keepdim=True) + eps)
    dg = (dy.to(DEV).double().reshape(rows, D) * xf * tau).sum(0)
    assert rel_l2(tg.grad, dg) <= 1e-4


def test_rms_norm_empty_and_deterministic():
    """No rows: empty output, zero dgain. Two backward passes give identical
    bits (fixed-order dgain reduction)."""
    x = torch.zeros((0, 768), dtype=torch.bfloat16, device=DEV, requires_grad=True)
    g = torch.ones(768, device=DEV, requires_grad=True)
    y = rms_norm(x, g)
    y.sum().backward()
    assert y.shape == (0, 768) and torch.count_nonzero(g.grad) == 0
    rng = np.random.default_rng(3)
    x = _randn(rng, (4096, 1024), "bf16").to(DEV)
    dy = _randn(rng, (4096, 1024), "bf16").to(DEV)
    grads = []
    for _ in range(2):
        g = torch.ones(1024, device=DEV, requires_grad=True)
        rms_norm(x, g).backward(dy)
        grads.append(g.grad.clone())
    assert torch.equal(grads[0], grads[1])


def _alu_inputs(rng, n, dtype):
    """Random values of scale 4 plus the reference test's grid (-40..40)
    and far tails, so both branches of 1 + u and both limits are exercised."""
    grid = np.linspace(-40, 40, 2001)
    tails = np.array([-1e6, -1e3, -60.0, 0.0, 60.0, 1e3, 1e6])
    vals = np.concatenate([grid, tails, 4 * rng.standard_normal(n - grid.size - tails.size)])
    return torch.from_numpy(vals.astype(np.float32)).to(_tdt(dtype))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("beta", [1.0, 0.5, 0.8])
@pytest.mark.parametrize("n", [4096, 4099, 5000])
def test_alu_output_and_vjp(dtype, beta, n):
    """Ragged sizes (4099, 5000 % 8 = 0 but 5000 % 16 != 0) take the tail path."""
    rng = np.random.default_rng(n)
    x = _alu_inputs(rng, n, dtype)
    dy = _randn(rng, (n,), dtype)
    tx = x.to(DEV).requires_grad_(True)
    y = alu(tx, beta)
    y.backward(dy.to(DEV))
    torch.cuda.synchronize()
    _check(dtype)(y, OE.alu(to_np(x), beta, dtype), what="y")
    _check(dtype)(tx.grad, OE.alu_vjp(to_np(x), to_np(dy), beta, dtype), what="dx")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", [(3, 7, 40), (2, 2048, 2688)])
def test_alu_glu_output_and_vjp(dtype, shape):
    """(3, 7, 40): 840 elements, a ragged vector tail for f32 and bf16; (2,
    2048, 2688): the 350M feed-forward width, oracle on a slice."""
    rng = np.random.default_rng(sum(shape))
    beta = 1.0
    gate = _randn(rng, shape, dtype)
    up = _randn(rng, shape, dtype, 2.0)
    dout = _randn(rng, shape, dtype)
    tgt = gate.to(DEV).requires_grad_(True)
    tup = up.to(DEV).requires_grad_(True)
    out = alu_glu(tgt, tup, beta)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    sl = (slice(0, 1), slice(0, 64)) if shape[1] > 64 else (slice(None),)
    g, u, d = to_np(gate[sl]), to_np(up[sl]), to_np(dout[sl])
    _check(dtype)(out[sl], OE.alu_glu(g, u, beta, dtype), what="out")
    want_dg, want_du = OE.alu_glu_vjp(g, u, d, beta, dtype)
    _check(dtype)(tgt.grad[sl], want_dg, what="dgate")
    _check(dtype)(tup.grad[sl], want_du, what="dup")


def test_alu_glu_equals_unfused_ops():
    """The fused product is the unfused graph gate * alu(up) with the same
    bf16 roundings: outputs and both gradients agree bit for bit."""
    rng = np.random.default_rng(11)
    shape = (4096, 2688)
    gate = _randn(rng, shape, "bf16").to(DEV)
    up = _randn(rng, shape, "bf16", 2.0).to(DEV)
    dout = _randn(rng, shape, "bf16").to(DEV)
    g1, u1 = gate.clone().requires_grad_(True), up.clone().requires_grad_(True)
    fused = alu_glu(g1, u1, 0.8)
    fused.backward(dout)
    g2, u2 = gate.clone().requires_grad_(True), up.clone().requires_grad_(True)
    unfused = g2 * alu(u2, 0.8)
    unfused.backward(dout)
    torch.cuda.synchronize()
    assert torch.equal(fused, unfused)
    assert torch.equal(g1.grad, g2.grad)
    assert torch.equal(u1.grad, u2.grad)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_glu_packed_alu_equals_alu_glu(dtype):
    """[gate | up] from one GEMM: the packed kernel gives alu_glu's outputs
    and gradients bit for bit, the gradient packed as [dgate | dup]."""
    from algebraic_amd.algebraic import glu_packed
    rng = np.random.default_rng(21)
    rows, f = 3000, 2688
    gu = _randn(rng, (rows, 2 * f), dtype, 2.0).to(DEV)
    dout = _randn(rng, (rows, f), dtype).to(DEV)
    a = gu.clone().requires_grad_(True)
    ya = glu_packed(a, "alu", 0.5)
    ya.backward(dout)
    gate = gu[:, :f].contiguous().requires_grad_(True)
    up = gu[:, f:].contiguous().requires_grad_(True)
    yb = alu_glu(gate, up, 0.5)
    yb.backward(dout)
    torch.cuda.synchronize()
    assert torch.equal(ya, yb)
    assert torch.equal(a.grad[:, :f], gate.grad) and torch.equal(a.grad[:, f:], up.grad)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("rows,f", [(37, 96), (2048, 2688)])
def test_glu_packed_silu_matches_oracle(dtype, rows, f):
    """The standard preset's SwiGLU on the packed projection (standard.py:12-13)."""
    from algebraic_amd.algebraic import glu_packed
    rng = np.random.default_rng(rows + f)
    gu = _randn(rng, (rows, 2 * f), dtype, 3.0)
    dout = _randn(rng, (rows, f), dtype)
    t = gu.to(DEV).requires_grad_(True)
    y = glu_packed(t, "silu")
    y.backward(dout.to(DEV))
    torch.cuda.synchronize()
    g, u, d = to_np(gu[:, :f]), to_np(gu[:, f:]), to_np(dout)
    _check(dtype)(y, OE.swiglu(g, u, dtype), what="y")
    want_dg, want_du = OE.swiglu_vjp(g, u, d, dtype)
    _check(dtype)(t.grad[:, :f], want_dg, what="dgate")
    _check(dtype)(t.grad[:, f:], want_du, what="dup")


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("with_gain", [True, False])
def test_add_rms_norm_equals_add_then_norm(dtype, with_gain):
    """The fused residual add + norm gives the unfused x + r and rms_norm's
    output bit for bit, and the same gradients (x's and r's are both the
    sum's): dx bit for bit, dgain to float32 reduction order."""
    from algebraic_amd.algebraic import add_rms_norm
    rng = np.random.default_rng(31)
    shape = (2, 300, 1024)
    x, r = _randn(rng, shape, dtype, 2.0).to(DEV), _randn(rng, shape, dtype).to(DEV)
    dsum, dy = _randn(rng, shape, dtype).to(DEV), _randn(rng, shape, dtype).to(DEV)
    gain = (torch.from_numpy((1 + 0.1 * rng.standard_normal(1024)).astype(np.float32)).to(DEV)
            if with_gain else None)
    outs, grads = [], []
    for fused in (True, False):
        tx, tr = x.clone().requires_grad_(True), r.clone().requires_grad_(True)
        tg = gain.clone().requires_grad_(True) if with_gain else None
        if fused:
            s, y = add_rms_norm(tx, tr, tg)
        else:
            s = tx + tr
            y = rms_norm(s, tg)
        torch.autograd.backward((s, y), (dsum, dy))
        outs.append((s.detach(), y.detach()))
        grads.append((tx.grad, tr.grad, tg.grad if with_gain else None))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])
    if with_gain:
        assert rel_l2(grads[0][2], grads[1][2]) <= 1e-6
