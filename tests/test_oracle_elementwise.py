"""Pins for the elementwise oracle (no GPU).

``oracle.elementwise`` restates rms_norm, alu (with the reference's
negative-tail form of 1 + u and its custom VJP) and the alu_glu product. These
tests check it against what shares none of that code: the closed form of the
reference's own test (test_components.py:71-78, same grid and tolerances),
central finite differences, an arcsinh form of the negative tail, torch float64
autograd, the norm's invariants, and torch's own bfloat16 arithmetic for the
rounding points.
"""

import numpy as np
import pytest
import torch

from oracle import elementwise as OE
from oracle import qknorm as OQ
from oracle.common import to_bf16


def _alu_closed(x, beta):
    return 0.5 * x * (1 + beta * x / np.sqrt(1 + (beta * x) ** 2))


@pytest.mark.parametrize("beta", [1.0, 0.5])
def test_alu_matches_closed_form(beta):
    """test_components.py:71-75: the grid linspace(-40, 40, 2001), rtol 1e-9."""
    x = np.linspace(-40, 40, 2001)
    np.testing.assert_allclose(OE.alu_parts(x, beta)[0], _alu_closed(x, beta), rtol=1e-9,
                               atol=1e-15)


@pytest.mark.parametrize("beta", [1.0, 0.5, 0.8])
def test_alu_derivative_matches_finite_differences_and_autograd(beta):
    """test_components.py:76-78 (grad of the closed form), here by central
    differences and torch float64 autograd of the closed form."""
    x = np.linspace(-40, 40, 2001)
    _, u, r = OE.alu_parts(x, beta)
    d = OE.alu_derivative(u, r)
    h = 1e-5 * np.maximum(1.0, np.abs(x))
    fd = (_alu_closed(x + h, beta) - _alu_closed(x - h, beta)) / (2 * h)
    np.testing.assert_allclose(d, fd, rtol=1e-7, atol=1e-10)
    t = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    y = 0.5 * t * (1 + beta * t / torch.sqrt(1 + (beta * t) ** 2))
    (g,) = torch.autograd.grad(y.sum(), t)
    np.testing.assert_allclose(d, g.numpy(), rtol=1e-9, atol=1e-12)
    dy = np.cos(x)
    np.testing.assert_allclose(OE.alu_vjp(x, dy, beta, "f64"), dy * g.numpy(), rtol=1e-9,
                               atol=1e-12)


def test_alu_negative_tail_keeps_relative_precision():
    """For x < 0, 1 + u = r / (|bx| + sqrt(1 + b^2 x^2)) = r exp(-asinh|bx|):
    the oracle keeps full relative precision where the closed form cancels."""
    x = -np.logspace(0, 12, 200)
    for beta in (1.0, 0.5):
        bz = beta * x
        r = 1 / np.sqrt(1 + bz * bz)
        want = 0.5 * x * r * np.exp(-np.arcsinh(np.abs(bz)))
        np.testing.assert_allclose(OE.alu_parts(x, beta)[0], want, rtol=1e-12)
    # the naive form loses everything far out (why the reference branches)
    assert _alu_closed(np.array([-1e9]), 1.0)[0] == 0.0
    assert OE.alu_parts(np.array([-1e9]), 1.0)[0][0] == pytest.approx(-2.5e-10, rel=1e-9)


def test_alu_special_values():
    """alu(0) = 0, alu(x) -> x for x >> 1, alu'(0) = 1/2, alu' -> 1 for x >> 1."""
    y, u, r = OE.alu_parts(np.array([0.0, 1e12]), 1.0)
    assert y[0] == 0.0 and y[1] == pytest.approx(1e12, rel=1e-12)
    d = OE.alu_derivative(u, r)
    assert d[0] == 0.5 and d[1] == pytest.approx(1.0, rel=1e-12)


def test_alu_glu_vjp_matches_autograd():
    rng = np.random.default_rng(5)
    gate, up, dout = (rng.standard_normal(4096) * 3 for _ in range(3))
    beta = 0.8
    tg = torch.tensor(gate, requires_grad=True)
    tu = torch.tensor(up, requires_grad=True)
    out = tg * (0.5 * tu * (1 + beta * tu / torch.sqrt(1 + (beta * tu) ** 2)))
    (out * torch.tensor(dout)).sum().backward()
    np.testing.assert_allclose(OE.alu_glu(gate, up, beta, "f64"), out.detach().numpy(),
                               rtol=1e-12, atol=1e-14)
    dg, du = OE.alu_glu_vjp(gate, up, dout, beta, "f64")
    np.testing.assert_allclose(dg, tg.grad.numpy(), rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(du, tu.grad.numpy(), rtol=1e-10, atol=1e-13)


def test_alu_glu_bf16_rounding_points_match_torch_bf16_ops():
    """The unfused bf16 graph: act = bf16(alu(up) in f32), out = gate * act
    as a bf16 multiply; the backward's dout * gate and dout * act are bf16
    multiplies too. torch's CPU bf16 ops round each product once, as XLA's do."""
    rng = np.random.default_rng(6)
    gate, up, dout = (torch.from_numpy(rng.standard_normal(8192).astype(np.float32)).bfloat16()
                      for _ in range(3))
    beta = 1.0
    act = torch.from_numpy(OE.alu_parts(up.double().numpy(), beta)[0].astype(np.float32)).bfloat16()
    out = gate * act
    want = OE.alu_glu(gate.double().numpy(), up.double().numpy(), beta, "bf16")
    np.testing.assert_array_equal(out.double().numpy(), want)
    dg, du = OE.alu_glu_vjp(gate.double().numpy(), up.double().numpy(), dout.double().numpy(),
                            beta, "bf16")
    np.testing.assert_array_equal((dout * act).double().numpy(), dg)
    gact = (dout * gate).double().numpy()
    _, u, r = OE.alu_parts(up.double().numpy(), beta)
    np.testing.assert_array_equal(to_bf16(gact * OE.alu_derivative(u, r)), du)


@pytest.mark.parametrize("with_gain", [False, True])
@pytest.mark.parametrize("eps", [1e-5, 1e-2])
def test_rms_norm_vjp_matches_autograd(with_gain, eps):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((6, 768)) * 2
    x[1] = 0.0
    gain = 1 + 0.1 * rng.standard_normal(768) if with_gain else None
    dy = rng.standard_normal((6, 768))
    tx = torch.tensor(x, requires_grad=True)
    tg = torch.tensor(gain, requires_grad=True) if with_gain else None
    tau = torch.rsqrt((tx * tx).mean(-1, keepdim=True) + eps)
    y = tx * tau * (tg if with_gain else 1.0)
    (y * torch.tensor(dy)).sum().backward()
    np.testing.assert_allclose(OE.rms_norm(x, gain, eps, "f64"), y.detach().numpy(), rtol=1e-13)
    dx, dg = OE.rms_norm_vjp(x, gain, dy, eps, "f64")
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-10, atol=1e-12)
    if with_gain:
        np.testing.assert_allclose(dg, tg.grad.numpy(), rtol=1e-6)
    else:
        assert dg is None


def test_rms_norm_invariants():
    """Unit RMS at eps -> 0, scale invariance, constant and zero rows, and
    agreement with the QK-norm oracle (the same function at D = 64)."""
    rng = np.random.default_rng(8)
    x = rng.standard_normal((5, 1024))
    y = OE.rms_norm(x, None, 1e-300, "f64")
    np.testing.assert_allclose(np.mean(y * y, -1), 1.0, rtol=1e-12)
    np.testing.assert_allclose(OE.rms_norm(7.5 * x, None, 1e-300, "f64"), y, rtol=1e-12)
    c = np.full((1, 768), 0.25)
    np.testing.assert_allclose(OE.rms_norm(c, None, 1e-5, "f64"), 0.25 / np.sqrt(0.0625 + 1e-5),
                               rtol=1e-14)
    assert not OE.rms_norm(np.zeros((2, 64)), None, 1e-5, "f64").any()
    g = 0.5 + rng.random(64)
    x64 = rng.standard_normal((9, 64))
    np.testing.assert_array_equal(OE.rms_norm(x64, g, 1e-5, "f32"), OQ.forward(x64, g, 1e-5, "f32"))
    # dx of a scale-invariant map is orthogonal to x (eps -> 0): sum(dx * x) = 0
    dx, _ = OE.rms_norm_vjp(x, None, rng.standard_normal(x.shape), 1e-300, "f64")
    np.testing.assert_allclose(np.sum(dx * x, -1), 0.0, atol=1e-10)


def test_swiglu_oracle_matches_autograd():
    """In float64 (no roundings) the SwiGLU oracle and its VJP are torch
    autograd of gate * up * sigmoid(up)."""
    rng = np.random.default_rng(12)
    gate, up, dout = (rng.standard_normal(2048) * 3 for _ in range(3))
    tg = torch.tensor(gate, requires_grad=True)
    tu = torch.tensor(up, requires_grad=True)
    out = tg * tu * torch.sigmoid(tu)
    (out * torch.tensor(dout)).sum().backward()
    np.testing.assert_allclose(OE.swiglu(gate, up, "f64"), out.detach().numpy(), rtol=1e-12,
                               atol=1e-14)
    dg, du = OE.swiglu_vjp(gate, up, dout, "f64")
    np.testing.assert_allclose(dg, tg.grad.numpy(), rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(du, tu.grad.numpy(), rtol=1e-10, atol=1e-13)
