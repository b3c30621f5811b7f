"""The optimizers on the GPU against the float64 oracle: Newton-Schulz as
batched GEMMs over layer-stacked weights, in float32 (tight) and bfloat16
(the default; each product's inputs rounded to bf16)."""

import numpy as np
import pytest
import torch

from _tol import rel_l2
from algebraic_amd import optimizers as O
from oracle import optimizers as OO

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("ns_dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 3e-2)])
@pytest.mark.parametrize("shape", [(24, 1024, 1024), (24, 1024, 2688), (24, 2688, 1024)])
def test_newton_schulz_at_model_shapes(ns_dtype, tol, shape):
    """The 350M model's stacked w_q/w_o, w_g/w_u and w_d shapes."""
    g = torch.Generator(device=DEV).manual_seed(0)
    G = torch.randn((2,) + shape[1:], generator=g, device=DEV)
    X = O.newton_schulz_5(G, ns_dtype=ns_dtype)
    torch.cuda.synchronize()
    want = OO.newton_schulz_5(G.double().cpu().numpy())
    assert rel_l2(X, want) <= tol


def test_muon_adamw_step_on_gpu_matches_oracle():
    rng = np.random.default_rng(4)
    shapes = {"embed": (97, 64), "final_gain": (64,)}
    lay = {"w_q": (2, 64, 64), "w_g": (2, 64, 96), "w_d": (2, 96, 64), "ln1": (2, 64)}
    params = {k: torch.tensor(rng.standard_normal(s), dtype=torch.float32, device=DEV)
              for k, s in shapes.items()}
    params["layers"] = {k: torch.tensor(rng.standard_normal(s), dtype=torch.float32, device=DEV)
                        for k, s in lay.items()}
    flat = {k: params[k].double().cpu().numpy() for k in shapes}
    flat.update({k: params["layers"][k].double().cpu().numpy() for k in lay})
    decay = {k: k.startswith("w_") or k == "embed" for k in flat}
    muon = {k: k.startswith("w_") for k in flat}
    mask = {"embed": True, "final_gain": False, "layers": {k: k.startswith("w_") for k in lay}}
    init_fn, step_fn = O.get_optimizer("muon_adamw", 2e-3)
    state = init_fn(params)
    m = {k: np.zeros_like(a) for k, a in flat.items()}
    v = {k: np.zeros_like(a) for k, a in flat.items()}
    for s in range(2):
        gr = {k: rng.standard_normal(a.shape) for k, a in flat.items()}
        gt = {k: torch.tensor(gr[k], dtype=torch.float32, device=DEV) for k in shapes}
        gt["layers"] = {k: torch.tensor(gr[k], dtype=torch.float32, device=DEV) for k in lay}
        p0 = {k: a.copy() for k, a in flat.items()}
        params, state = step_fn(s, params, gt, state, mask)
        flat, m, v = OO.step("muon_adamw", s, flat, gr, m, v, decay, muon, lr=2e-3)
        torch.cuda.synchronize()
        got = {k: params[k].double().cpu().numpy() for k in shapes}
        got.update({k: params["layers"][k].double().cpu().numpy() for k in lay})
        for k in flat:
            # compare the updates: bf16 Newton-Schulz on Muon leaves; on the
            # others the float32 parameter itself (|p| ~ 1, one ulp ~ 1e-7)
            # rounds an update of ~1e-4 to ~1e-3 relative
            tol = 3e-2 if muon[k] else 2e-3
            assert rel_l2(got[k] - p0[k], flat[k] - p0[k]) <= tol, k
        flat = got


@pytest.mark.parametrize("n", [0, 1, 7, 4096, 1000003])
def test_muon_elementwise_kernels(n):
    """algx_muon_momentum / algx_muon_apply against optimizers.py:200-204 in
    float64 (float32 state: a few ulp), with n not a multiple of the 4-element
    vector and o in bf16 and float32."""
    rng = np.random.default_rng(n)
    g64, m64, p64 = (rng.standard_normal(n) for _ in range(3))
    g = torch.tensor(g64, dtype=torch.float32, device=DEV)
    m = torch.tensor(m64, dtype=torch.float32, device=DEV)
    mu = 0.95
    look = O._muon_momentum(g, m, mu)
    gf, mf = g64.astype(np.float32).astype(np.float64), m64.astype(np.float32).astype(np.float64)
    m_want = mu * mf + (1 - mu) * gf
    look_want = (1 - mu) * gf + mu * m_want
    np.testing.assert_allclose(m.double().cpu().numpy(), m_want, rtol=0, atol=1e-6)
    np.testing.assert_allclose(look.double().cpu().numpy(), look_want, rtol=0, atol=1e-6)
    for odt in (torch.bfloat16, torch.float32):
        p = torch.tensor(p64, dtype=torch.float32, device=DEV)
        o = look.to(odt)
        decay, step = 1.0 - 2e-3 * 0.1, 2e-3 * 1.62
        O._muon_apply(p, o, decay, step)
        want = p64.astype(np.float32).astype(np.float64) * decay - step * o.double().cpu().numpy()
        np.testing.assert_allclose(p.double().cpu().numpy(), want, rtol=0, atol=2e-6)


@pytest.mark.parametrize("shape", [(3, 5, 7), (2, 64, 96), (96, 1024, 1024), (1, 1, 3)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_ns_normalize_kernel(shape, out_dtype):
    """algx_ns_normalize against optimizers.py:44-45 in float64: X / sqrt(sum
    X^2 + eps) per matrix, on the vector path (extents a multiple of 4) and
    the scalar one, written in bf16 (within one bf16 rounding) or float32."""
    g = torch.Generator(device=DEV).manual_seed(sum(shape))
    X = torch.randn(shape, generator=g, device=DEV) * 3.0
    out = torch.empty(shape, dtype=out_dtype, device=DEV)
    O._normalize_into(X, out, 1e-7)
    x64 = X.double().cpu()
    want = x64 / torch.sqrt((x64 * x64).sum(dim=(-2, -1), keepdim=True) + 1e-7)
    got = out.double().cpu()
    tol = 2.0 ** -8 if out_dtype == torch.bfloat16 else 4e-6
    assert float(((got - want).abs() / want.abs().clamp_min(1e-30)).max()) <= tol


@pytest.mark.parametrize("n", [1, 5, 4096, 51513])
def test_adamw_step_kernel(n):
    """algx_adamw_step against optimizers.py:222-226 in float64 from the same
    float32 state (a few float32 ulp)."""
    rng = np.random.default_rng(n + 1)
    p64, g64, m64 = (rng.standard_normal(n) for _ in range(3))
    v64 = rng.random(n) * 0.1
    ts = [torch.tensor(a, dtype=torch.float32, device=DEV) for a in (p64, g64, m64, v64)]
    b1, b2, eps, lr, decay = 0.9, 0.95, 1e-8, 2e-3, 1.0 - 2e-3 * 0.1
    t = 3.0
    c1, c2 = 1.0 - b1 ** t, 1.0 - b2 ** t
    O._adamw_step(ts[0], ts[1], ts[2], ts[3], b1, b2, c1, c2, eps, decay, lr)
    p, g, m, v = (a.astype(np.float32).astype(np.float64) for a in (p64, g64, m64, v64))
    m = b1 * m + (1 - b1) * g
    v = b2 * v + (1 - b2) * g * g
    p = p * decay - lr * (m / c1) / (np.sqrt(v / c2) + eps)
    np.testing.assert_allclose(ts[2].double().cpu().numpy(), m, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(ts[3].double().cpu().numpy(), v, rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(ts[0].double().cpu().numpy(), p, rtol=1e-6, atol=1e-6)
