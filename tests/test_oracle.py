"""Pins for the CPU oracle (no GPU): closed forms, textbook formulations,
float64 autograd, finite differences and the reference's known answers.

The oracle restates the reference kernels' code paths (rho, int_pow, inverse
statistics, max shifts, the closed-form tile VJP, the sink gradient, the
guard); these tests check it against formulations that share none of that
code: softmax over the compressed logits ``n*asinh(s/c)`` (the identity of the
reference's test_components.py:28-41), torch float64 autograd of that softmax,
and constants quoted by the reference's own tests.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import head as OH
from oracle import qknorm as OQ
from oracle.common import (bounded_radical, inv_root, ipow, rho_exact, rho_fast, root, tiled_rho,
                           to_bf16)

# ---------------------------------------------------------------------------
# elementwise algebra
# ---------------------------------------------------------------------------


def test_rho_identities():
    """test_components.py:18-26: rho = exp(asinh), rho(x) rho(-x) = 1, oplus law."""
    x = np.linspace(-50, 50, 1001)
    y = np.linspace(-3, 7, 1001)
    np.testing.assert_allclose(rho_exact(x)[0], np.exp(np.arcsinh(x)), rtol=1e-12)
    np.testing.assert_allclose(rho_exact(x)[0] * rho_exact(-x)[0], 1.0, rtol=1e-12)
    oplus = x * np.sqrt(1 + y * y) + y * np.sqrt(1 + x * x)
    np.testing.assert_allclose(rho_exact(x)[0] * rho_exact(y)[0], rho_exact(oplus)[0], rtol=1e-10)
    # r = d log rho / dx = 1/sqrt(1+x^2) (derivative of asinh)
    np.testing.assert_allclose(rho_exact(x)[1], 1 / np.sqrt(1 + x * x), rtol=1e-14)
    # fast rho agrees on the positive side
    xp = np.linspace(0, 50, 101)
    np.testing.assert_allclose(rho_fast(xp)[0], np.exp(np.arcsinh(xp)), rtol=1e-13)


def test_rho_known_answers():
    """test_e2e_requirements.py:1000-1016 in float32."""
    v = rho_exact(np.float32(-1e6))[0]
    assert np.isfinite(v) and v > 0
    assert math.isclose(float(v), 1.0 / (1e6 + math.sqrt(1.0 + 1e12)), rel_tol=1e-3)
    assert rho_exact(np.float32(1e6))[0] > 1e6


def test_bounded_radical_pins():
    """radical.py:13-38. On |x| <= 1 the polynomials approximate rho(x) and
    r = 1/sqrt(1+x^2) (the fit's error: < 5e-5 and < 2e-4 relative); at x = 0
    they give their constant terms (coefficient order); any |x| > 1 in the
    array sends all of it down the exact stable radical (one cond per call)."""
    x = np.linspace(-1.0, 1.0, 4001)
    rp, rr = bounded_radical(x)
    re, ri = rho_exact(x)
    assert np.max(np.abs(rp - re) / re) < 5e-5
    assert np.max(np.abs(rr - ri) / ri) < 2e-4
    r0, s0 = bounded_radical(np.zeros(3))
    assert np.allclose(r0, np.float32(1.0000227161113386)) and np.allclose(s0, np.float32(.9998514827226793))
    # the sqrt(1+t) fit at t = 1 is sqrt(2), the rsqrt fit 1/sqrt(2) (both to the fit error)
    assert abs(bounded_radical(np.array([1.0]))[0][0] - (1 + math.sqrt(2))) < 1e-4
    mixed = np.array([0.25, -0.5, 1.5])
    np.testing.assert_array_equal(bounded_radical(mixed)[0], rho_exact(mixed)[0])
    # per (head, tile): one large score makes only its own tile of its own head exact
    xs = np.full((1, 2, 4, 4), 0.3)
    xs[0, 1, 0, 3] = 2.0
    rh, _ = tiled_rho(xs, True, True, 2, 2)
    poly_val = bounded_radical(np.array([0.3]))[0][0]
    exact_val = rho_exact(np.array([0.3]))[0][0]
    assert poly_val != exact_val
    np.testing.assert_array_equal(rh[0, 0], poly_val)
    np.testing.assert_array_equal(rh[0, 1, 0:2, 2:4][rh[0, 1, 0:2, 2:4] < 1.5], exact_val)
    np.testing.assert_array_equal(rh[0, 1, 2:4], poly_val)
    np.testing.assert_array_equal(rh[0, 1, 0:2, 0:2], poly_val)


def test_ipow_and_roots():
    x = np.linspace(0.1, 3, 50)
    for n in (1, 2, 3, 8, 16, 32):
        np.testing.assert_allclose(ipow(x, n), x ** n, rtol=1e-13)
    for n in (2, 4, 8, 16, 32):
        np.testing.assert_allclose(inv_root(x, n), x ** (-1.0 / n), rtol=1e-13)
        assert math.isclose(root(1e37, n), 1e37 ** (1.0 / n), rel_tol=1e-12)
    with pytest.raises(ValueError):
        ipow(x, 0)


# ---------------------------------------------------------------------------
# variants and guard constants
# ---------------------------------------------------------------------------


def test_make_variant_constants():
    """Clamps quoted for flash.py:747-748: T=2048 n=16 -> 63.75, T=256 -> 72.58."""
    v = OA.make_variant("asinh", 16, 8.0, 2048)
    assert abs(v.clamp - 63.75) < 5e-3 and not v.shift and v.inv_stat and v.fast_rho
    assert abs(OA.make_variant("asinh", 16, 8.0, 256).clamp - 72.58) < 5e-3
    # rho(clamp)^n (T+1) = 1e37 exactly, the defining equation of the clamp
    for n, T in ((8, 512), (16, 2048), (32, 300)):
        v = OA.make_variant("asinh", n, 1.0, T)
        assert math.isclose(rho_exact(v.clamp)[0] ** n * (T + 1), 1e37, rel_tol=1e-9)
    # n=32 at T=2048 has clamp < 20 and defaults to the shifted kernel
    assert OA.make_variant("asinh", 32, 8.0, 2048).shift
    bound, vmax = OA.guard_bounds(OA.make_variant("asinh", 16, 8.0, 2048), 2048, False)
    assert bound == 16.0 and vmax == 1e8
    with pytest.raises(ValueError, match="power of two"):
        OA.make_variant("asinh", 12)
    with pytest.raises(ValueError, match="positive and finite"):
        OA.make_variant("asinh", 16, -1.0)
    with pytest.raises(ValueError, match="requires shift=False"):
        OA.make_variant("asinh", 16, 8.0, shift=True, inv_stat=True)
    with pytest.raises(ValueError, match="unknown attention"):
        OA.make_variant("relu")


# ---------------------------------------------------------------------------
# textbook attention (independent formulation) in torch float64
# ---------------------------------------------------------------------------


def textbook_attention(q, k, v, sink_logit, kind, n, c):
    """softmax over n*asinh(s/c) (or s for softmax) with the sink as one extra logit."""
    q, k, v = (torch.as_tensor(a, dtype=torch.float64) for a in (q, k, v))
    B, H, T, D = q.shape
    s = q @ k.transpose(-1, -2) / math.sqrt(D)
    logits = n * torch.asinh(s / c) if kind == "asinh" else s
    mask = torch.tril(torch.ones(T, T, dtype=torch.bool))
    logits = logits.masked_fill(~mask, float("-inf"))
    if sink_logit is not None:
        b = torch.as_tensor(sink_logit, dtype=torch.float64).reshape(1, -1, 1, 1).expand(B, H, T, 1)
        b = n * torch.asinh(b / c) if kind == "asinh" else b
        p = torch.softmax(torch.cat([logits, b], -1), -1)[..., :T]
    else:
        p = torch.softmax(logits, -1)
    return p @ v


def _inputs(shape, seed, scale=1.5, sink=True):
    rng = np.random.default_rng(seed)
    q, k, v, g = (rng.standard_normal(shape).astype(np.float32).astype(np.float64) for _ in range(4))
    sk = (rng.standard_normal(shape[1]) * 0.5).astype(np.float32).astype(np.float64) if sink else None
    return q * scale, k * scale, v, g, sk


CASES = [("asinh", 16, 16.0, True, True, False), ("asinh", 16, 16.0, True, True, True),
         ("asinh", 16, 16.0, True, False, True), ("asinh", 16, 16.0, False, False, True),
         ("asinh", 8, 1.0, True, True, False), ("asinh", 32, 8.0, False, True, True),
         ("asinh", 16, 8.0, True, None, None), ("softmax", 16, 16.0, True, None, None),
         ("softmax", 16, 16.0, False, None, None)]


def _oracle_exact(q, k, v, sk, kind, n, c, shift, fast, guard=False, do=None):
    """Oracle kernel path in float64 (no dtype rounding), scale folded exactly."""
    B, H, T, D = q.shape
    var = OA.make_variant(kind, n, c, T, shift, fast)
    unit = 1.0 if kind == "softmax" else c
    scale = 1 / (math.sqrt(D) * unit)
    sink = None if sk is None else np.broadcast_to(sk.reshape(-1), (H,)) / unit
    qs = q * scale
    if guard and kind == "asinh":
        low, high = OA.low_high(var)
        var = low if OA.guard_in_range(qs, k, v, sink, var, sk is not None) else high
    o, o_res, stat = OA.forward(qs, k, v, sink, var, sk is not None, "f64")
    if do is None:
        return o
    dq, dk, dv, dsink, _ = OA.backward(qs, k, v, sink, o_res, stat, do, var, sk is not None, "f64")
    return o, (dq * scale, dk, dv, None if sk is None else dsink / unit)


@pytest.mark.parametrize("kind,n,c,with_sink,shift,fast", CASES)
@pytest.mark.parametrize("guard", [False, True])
def test_oracle_forward_and_vjp_match_textbook(kind, n, c, with_sink, shift, fast, guard):
    """Oracle kernel numerics (every variant) == textbook softmax and its autograd VJP."""
    if guard and kind != "asinh":
        pytest.skip("guard applies to asinh only")
    shape = (2, 3, 24, 16)
    q, k, v, g, sk = _inputs(shape, 7, sink=with_sink)
    o, grads = _oracle_exact(q, k, v, sk, kind, n, c, shift, fast, guard, do=g)
    tq, tk, tv = (torch.tensor(a, requires_grad=True) for a in (q, k, v))
    ts = torch.tensor(sk, requires_grad=True) if with_sink else None
    ref = textbook_attention(tq, tk, tv, ts, kind, n, c)
    np.testing.assert_allclose(o, ref.detach().numpy(), rtol=1e-9, atol=1e-12)
    (ref * torch.tensor(g)).sum().backward()
    want = [tq.grad, tk.grad, tv.grad] + ([ts.grad] if with_sink else [])
    for got, w in zip(grads, want):
        w = w.numpy()
        np.testing.assert_allclose(got, w, rtol=1e-8, atol=1e-10 * np.abs(w).max())


def test_oracle_vjp_finite_differences_with_clamp_binding():
    """Unguarded shift=False clamps scores at ``clamp``; the VJP is the derivative
    of the clipped function (zero above the cap, flash.py:357-360). Checked by
    central differences of the oracle forward on a case where some scores bind."""
    rng = np.random.default_rng(3)
    B, H, T, D = 1, 1, 6, 4
    n, c = 8, 1.0
    var = OA.make_variant("asinh", n, c, T, shift=False)
    qs = rng.standard_normal((B, H, T, D))
    k = rng.standard_normal((B, H, T, D))
    qs[0, 0, 3] *= 0.0
    qs[0, 0, 3, 0] = 4.0 * var.clamp      # row 3 scores bind for k[...,0] > 0.25
    k[0, 0, :, 0] = np.abs(k[0, 0, :, 0]) + 0.5
    v = rng.standard_normal((B, H, T, D))
    g = rng.standard_normal((B, H, T, D))
    sink = np.array([0.3])

    def f(qs_, k_, v_, sink_):
        return np.sum(OA.forward(qs_, k_, v_, sink_, var, True, "f64")[0] * g)

    o, o_res, stat = OA.forward(qs, k, v, sink, var, True, "f64")
    dq, dk, dv, dsink, _ = OA.backward(qs, k, v, sink, o_res, stat, g, var, True, "f64")
    eps = 1e-6
    for arr, grad in ((qs, dq), (k, dk), (v, dv), (sink, dsink)):
        num = np.zeros_like(arr)
        it = np.nditer(arr, flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            old = arr[idx]
            arr[idx] = old + eps
            fp = f(qs, k, v, sink)
            arr[idx] = old - eps
            fm = f(qs, k, v, sink)
            arr[idx] = old
            num[idx] = (fp - fm) / (2 * eps)
        np.testing.assert_allclose(grad, num, rtol=1e-5, atol=1e-7)
    assert np.any(np.minimum(OA._scores(qs, k), 1e9) >= var.clamp)   # the clamp did bind


def test_explicit_clipping_vjp_is_zero_above_cap():
    """test_flash_kernel_tpu.py:122-138 restated: saturated scores and sink give exactly zero grads."""
    shape = (1, 1, 256, 64)
    q = np.full(shape, math.sqrt(1000), np.float32).astype(np.float64)
    rng = np.random.default_rng(39)
    v = rng.standard_normal(shape).astype(np.float32).astype(np.float64)
    g = rng.standard_normal(shape).astype(np.float32).astype(np.float64)
    res = OA.flash_attention(q, q, v, np.full((1,), 1000.0), kind="asinh", n=16, c=8.0,
                             shift=False, range_guard=False, dtype="f32", do=g)
    dq, dk, dv, dsink = res.grads
    assert np.all(dq == 0) and np.all(dk == 0) and np.all(dsink == 0)


def test_guard_decisions():
    """flash.py:840-849: typical inputs are in range; the tails are not."""
    shape = (1, 2, 256, 64)
    q, k, v, _, _ = _inputs(shape, 1, scale=1.0, sink=False)
    var = OA.make_variant("asinh", 16, 8.0, 256)
    qs = q / 64.0
    assert OA.guard_in_range(qs, k, v, None, var, False)
    assert OA.guard_in_range(qs, k, v, np.array([0.1, -2.0]), var, True)
    assert not OA.guard_in_range(qs, k, v, np.array([0.1, 20.0]), var, True)
    big = np.full(shape, math.sqrt(1000))
    assert not OA.guard_in_range(big / 64.0, big, v, None, var, False)
    assert not OA.guard_in_range(qs, k, v * 2e8, None, var, False)


@pytest.mark.parametrize("score_sign", [-1.0, 1.0])
@pytest.mark.parametrize("with_sink", [False, True])
@pytest.mark.parametrize("magnitude", [1000.0, 1e7])
def test_guarded_tail_matches_dense(score_sign, with_sink, magnitude):
    """test_flash_kernel_tpu.py:100-119 restated on the oracle (float32 rounding)."""
    shape = (1, 1, 256, 64)
    q = np.full(shape, math.sqrt(magnitude), np.float32).astype(np.float64)
    k = q * score_sign
    v = np.random.default_rng(29).standard_normal(shape).astype(np.float32).astype(np.float64)
    sink = np.zeros((1,)) if with_sink else None
    res = OA.flash_attention(q, k, v, sink, kind="asinh", n=16, c=8.0, range_guard=True,
                             dtype="f32", do=np.ones(shape))
    assert res.in_range is False and res.variant.shift
    ref = OA.dense_asinh_attention(q, k, v, n=16, c=8.0, sink_logit=sink)
    assert np.isfinite(res.o).all()
    np.testing.assert_allclose(res.o, ref, atol=2e-3, rtol=2e-3)
    assert all(np.isfinite(x).all() for x in res.grads[:3])


def test_dense_asinh_matches_textbook():
    q, k, v, _, sk = _inputs((2, 3, 20, 8), 11)
    for n, c in ((16, 8.0), (8, 1.0), (32, 4.0)):
        got = OA.dense_asinh_attention(q, k, v, n=n, c=c, sink_logit=sk)
        want = textbook_attention(q, k, v, sk, "asinh", n, c).numpy()
        np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-13)
    got = OA.dense_softmax_attention(q, k, v, sink_logit=sk)
    np.testing.assert_allclose(got, textbook_attention(q, k, v, sk, "softmax", 1, 1).numpy(),
                               rtol=1e-10, atol=1e-13)


def test_dense_weights_survive_huge_scores():
    """test_components.py:39-40: the max shift keeps 1e6-scaled scores finite."""
    q, k, v, _, _ = _inputs((1, 2, 7, 8), 5, sink=False)
    out = OA.dense_asinh_attention(q * 1e3, k * 1e3, v, n=16, c=16.0)
    assert np.isfinite(out).all()


def test_bf16_rounding_helper():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -9, -3.14159, 1e-40, 65504.0])
    r = to_bf16(x)
    assert r[0] == 1.0 and r[1] == 1.0            # tie -> even
    assert r[2] == 1.0 + 2 ** -7                    # tie -> even (up)
    assert abs(r[3] + 3.140625) < 1e-12


# ---------------------------------------------------------------------------
# fused head
# ---------------------------------------------------------------------------


def test_head_clamp_constants():
    """fused_head.py:273: V=50304 gives 3632.8 (n=8) and 30.14 (n=16); ~31 for 32768, n=16."""
    assert abs(OH.head_clamp(50304, 8) - 3632.8) < 0.05
    assert abs(OH.head_clamp(50304, 16) - 30.14) < 0.005
    assert 30.5 < OH.head_clamp(32768, 16) < 31.5


@pytest.mark.parametrize("kind,n,c", [("ce", 16, 16.0), ("alg_ce", 16, 16.0), ("alg_ce", 8, 2.0)])
def test_head_oracle_matches_textbook(kind, n, c):
    """Objective/telemetry and (dh, dE) of the restated kernel == textbook log-loss autograd.

    For alg_ce the reference's gradient is the exact gradient of the mean NLL of
    log_softmax(n*asinh(z/c)) (test_components.py:43-56); its telemetry is the
    target probability.
    """
    rng = np.random.default_rng(5)
    N, d, V = 12, 16, 37
    h = rng.standard_normal((N, d)) * 2
    e = rng.standard_normal((V, d)) * 0.8
    t = rng.integers(0, V, N)
    (obj, tel), (dh, de) = OH.fused_head(h, e, t, kind=kind, n=n, c=c, dtype="f64",
                                        embed_dtype="f64", g_obj=1.0)
    th, te = torch.tensor(h, requires_grad=True), torch.tensor(e, requires_grad=True)
    z = th @ te.T
    a = n * torch.asinh(z / c) if kind == "alg_ce" else z
    logp = torch.log_softmax(a, -1)[torch.arange(N), torch.tensor(t)]
    nll = -logp.mean()
    nll.backward()
    np.testing.assert_allclose(dh, th.grad.numpy(), rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(de, te.grad.numpy(), rtol=1e-9, atol=1e-12)
    if kind == "ce":
        assert math.isclose(obj, float(nll), rel_tol=1e-12)
        np.testing.assert_allclose(tel, -logp.detach().numpy(), rtol=1e-12)
    else:
        np.testing.assert_allclose(tel, np.exp(logp.detach().numpy()), rtol=1e-10)
        assert math.isclose(obj, float(np.mean(1 - np.exp(logp.detach().numpy()))), rel_tol=1e-10)
        np.testing.assert_allclose(np.log(tel), OH.dense_alg_logprob(h @ e.T, t, n, c), rtol=1e-9)


def test_head_padding_free_ragged_vocab():
    """Ragged V (not a tile multiple) is exact in the dense oracle: sums run over V only."""
    rng = np.random.default_rng(6)
    h, e = rng.standard_normal((8, 8)), rng.standard_normal((13, 8))
    t = rng.integers(0, 13, 8)
    (obj, tel), _ = OH.fused_head(h, e, t, kind="ce", dtype="f64")
    assert math.isclose(obj, OH.dense_ce(h @ e.T, t)[0], rel_tol=1e-12)


# ---------------------------------------------------------------------------
# QK RMS norm
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("eps", [1e-5, 1e-3])
def test_qknorm_matches_autograd(eps):
    rng = np.random.default_rng(181)
    x = 3 * rng.standard_normal((2, 3, 16, 64))
    x[0, 0, 0] = 0
    gain = 0.25 + 4 * rng.random(64)
    dy = rng.standard_normal(x.shape)
    y = OQ.forward(x, gain, eps, "f64")
    dx, dg = OQ.backward(x, gain, dy, eps, "f64")
    tx, tg = torch.tensor(x, requires_grad=True), torch.tensor(gain, requires_grad=True)
    ty = tx * torch.rsqrt((tx * tx).mean(-1, keepdim=True) + eps) * tg
    (ty * torch.tensor(dy)).sum().backward()
    np.testing.assert_allclose(y, ty.detach().numpy(), rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dg, tg.grad.numpy().astype(np.float32), rtol=1e-6)
    # RMS of the normalised rows is ~1 (gain 1)
    y1 = OQ.forward(x, np.ones(64), 0.0 + 1e-12, "f64").reshape(-1, 64)[1:]
    np.testing.assert_allclose(np.sqrt((y1 ** 2).mean(-1)), 1.0, rtol=1e-9)


def test_qknorm_validation_messages():
    """qk_norm.py:68-75."""
    assert OQ.validate((4, 64), 64, (64,), "bf16", "f32", 1024, 1024, 1e-5) is None
    assert "D=64" in OQ.validate((4, 32), 32, (32,), "bf16", "f32", 1024, 1024, 1e-5)
    assert "float32/BF16" in OQ.validate((4, 64), 64, (64,), "f16", "f32", 1024, 1024, 1e-5)
    assert "divisible" in OQ.validate((4, 64), 64, (64,), "bf16", "f32", 1000, 1024, 1e-5)
    assert "positive" in OQ.validate((4, 64), 64, (64,), "bf16", "f32", 1024, 1024, 0.0)
