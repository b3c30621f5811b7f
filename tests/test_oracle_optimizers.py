"""Pins for the optimizer oracle, and the torch optimizers (on the CPU)
against it (no GPU).

Newton-Schulz against the SVD polar factor U V^T and the reference's own
orthogonality check (test_e2e_requirements.py:1030-1039: max|O O^T - I| < 0.25
for a 64 x 64 Gaussian); the Adam-family step against torch.optim.AdamW; the
schedule against closed-form values.
"""

import math

import numpy as np
import pytest
import torch

from algebraic_amd import optimizers as O
from oracle import optimizers as OO


@pytest.mark.parametrize("shape", [(64, 64), (48, 80), (96, 40), (3, 32, 24)])
def test_newton_schulz_is_close_to_the_polar_factor(shape):
    rng = np.random.default_rng(1)
    G = rng.standard_normal(shape)
    X = OO.newton_schulz_5(G)
    U, s, Vt = np.linalg.svd(G, full_matrices=False)
    polar = U @ Vt * math.sqrt(max(1.0, shape[-2] / shape[-1]))
    sv = np.linalg.svd(X / math.sqrt(max(1.0, shape[-2] / shape[-1])), compute_uv=False)
    assert np.all(sv > 0.6) and np.all(sv < 1.25)          # quintic band, refined
    cos = np.sum(X * polar) / (np.linalg.norm(X) * np.linalg.norm(polar))
    assert cos > 0.99
    if shape == (64, 64):
        assert np.abs(X @ X.T - np.eye(64)).max() < 0.25
    if len(shape) == 2 and shape[0] > shape[1]:
        np.testing.assert_allclose(X, OO.newton_schulz_5(G.T).T * math.sqrt(shape[0] / shape[1]),
                                   rtol=1e-12, atol=1e-12)


def test_cosine_schedule_closed_form():
    f = O.make_cosine_schedule(2e-3, 1000, 0.02, 0.1)
    assert f(0) == pytest.approx(2e-3 / 20)            # t = 1 of 20 warmup steps
    assert f(19) == pytest.approx(2e-3)                # end of warmup: peak
    assert f(999) == pytest.approx(2e-4)               # end: min_lr_ratio * peak
    mid = 19 + (1000 - 20) / 2
    assert f(mid) == pytest.approx(2e-4 + 1.8e-3 * 0.5, rel=1e-9)
    for s in (0, 7, 19, 300, 999):
        assert f(s) == pytest.approx(OO.cosine_lr(s, 2e-3, 1000, 0.02, 0.1), rel=1e-12)


def test_adamw_step_matches_torch_adamw():
    """'muon_adamw' on a non-Muon leaf is AdamW; torch's own AdamW with the
    same lr (the schedule's value), betas, eps and decoupled decay agrees."""
    rng = np.random.default_rng(2)
    p0 = rng.standard_normal(100)
    grads = [rng.standard_normal(100) for _ in range(3)]
    lrs = [OO.cosine_lr(s, 1e-2, 1000, 0.02, 0.1) for s in range(3)]
    tp = torch.tensor(p0, requires_grad=True)
    opt = torch.optim.AdamW([tp], lr=lrs[0], betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    P, m, v = {"embed": p0}, {"embed": np.zeros(100)}, {"embed": np.zeros(100)}
    for s in range(3):
        for group in opt.param_groups:
            group["lr"] = lrs[s]
        tp.grad = torch.tensor(grads[s])
        opt.step()
        P, m, v = OO.step("muon_adamw", s, P, {"embed": grads[s]}, m, v, {"embed": True},
                          {"embed": False}, lr=1e-2)
    np.testing.assert_allclose(P["embed"], tp.detach().numpy(), rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("name", ["muon_adamw", "cadamw", "hybrid_muon_cadamw"])
def test_torch_optimizer_matches_oracle(name):
    """The package's step_fn (float32, Newton-Schulz in float32, on the CPU)
    against the float64 oracle over three steps of a small model-like tree."""
    rng = np.random.default_rng(3)
    shapes = {"embed": (40, 16), "final_gain": (16,)}
    lay = {"w_q": (2, 16, 16), "w_d": (2, 24, 16), "ln1": (2, 16), "sink": (2, 4)}
    params = {k: torch.tensor(rng.standard_normal(s), dtype=torch.float32) for k, s in shapes.items()}
    params["layers"] = {k: torch.tensor(rng.standard_normal(s), dtype=torch.float32)
                        for k, s in lay.items()}
    flat = {k: params[k].double().numpy() for k in shapes}
    flat.update({k: params["layers"][k].double().numpy() for k in lay})
    decay = {k: k.startswith("w_") or k == "embed" for k in flat}
    muon = {k: O.is_muon_param((k,), flat[k]) for k in flat}
    assert muon == {"embed": False, "final_gain": False, "w_q": True, "w_d": True, "ln1": False,
                    "sink": False}
    init_fn, step_fn = O.get_optimizer(name, 1e-2, ns_dtype=torch.float32)
    state = init_fn(params)
    mask = {"embed": True, "final_gain": False,
            "layers": {k: k.startswith("w_") for k in lay}}
    m = {k: np.zeros_like(a) for k, a in flat.items()}
    v = {k: np.zeros_like(a) for k, a in flat.items()}
    for s in range(3):
        g = {k: rng.standard_normal(a.shape) for k, a in flat.items()}
        gt = {k: torch.tensor(g[k], dtype=torch.float32) for k in shapes}
        gt["layers"] = {k: torch.tensor(g[k], dtype=torch.float32) for k in lay}
        params, state = step_fn(s, params, gt, state, mask)
        flat, m, v = OO.step(name, s, flat, g, m, v, decay, muon, lr=1e-2)
    got = {k: params[k].double().numpy() for k in shapes}
    got.update({k: params["layers"][k].double().numpy() for k in lay})
    for k in flat:
        np.testing.assert_allclose(got[k], flat[k], rtol=1e-4, atol=1e-5, err_msg=k)


def test_grouped_newton_schulz_equals_one_by_one():
    """Batching equal shapes (and transposed tall ones) changes nothing."""
    rng = np.random.default_rng(5)
    Gs = [torch.tensor(rng.standard_normal(s), dtype=torch.float32)
          for s in ((2, 16, 16), (2, 16, 40), (2, 40, 16), (3, 16, 16), (16, 40))]
    many = O.newton_schulz_many(Gs, ns_dtype=torch.float32)
    for G, got in zip(Gs, many):
        want = O.newton_schulz_5(G, ns_dtype=torch.float32)
        assert got.shape == G.shape
        np.testing.assert_allclose(got.numpy(), want.numpy(), rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(got.double().numpy(), OO.newton_schulz_5(G.double().numpy()),
                                   rtol=1e-4, atol=1e-5)
