"""CPU oracle: the reference's optimizers in float64 NumPy (test infrastructure only).

Restates src/algebraic/optimizers.py: ``newton_schulz_5`` (:27-64) on the
trailing two axes, the cosine schedule with linear warmup (:92-115) and one
step of 'muon_adamw', 'cadamw' and 'hybrid_muon_cadamw' (:118-246) on a flat
{name: array} parameter set. Pinned in tests/test_oracle_optimizers.py against
the SVD polar factor, torch.optim.AdamW and closed-form schedule values.
"""

import math

import numpy as np

F64 = np.float64


def newton_schulz_5(G, steps=5, eps=1e-7):
    a, b, c = 3.4445, -4.7750, 2.0315
    G = np.asarray(G, F64)
    M, N = G.shape[-2], G.shape[-1]
    transposed = M > N
    X = np.swapaxes(G, -2, -1) if transposed else G
    X = X / np.sqrt(np.sum(X * X, axis=(-2, -1), keepdims=True) + eps)
    for _ in range(steps):
        A = X @ np.swapaxes(X, -2, -1)
        X = a * X + (b * A + c * (A @ A)) @ X
    eye = np.eye(min(M, N))
    for _ in range(2):
        X = 0.5 * (3.0 * eye - X @ np.swapaxes(X, -2, -1)) @ X
    if transposed:
        X = np.swapaxes(X, -2, -1)
    return X * math.sqrt(max(1.0, M / N))


def cosine_lr(step, peak, total, warmup_fraction, min_ratio):
    warm = warmup_fraction if warmup_fraction >= 1 else max(1.0, float(round(warmup_fraction * total)))
    t = step + 1.0
    if t < warm:
        return peak * min(1.0, t / warm)
    prog = min(max((t - warm) / max(1.0, total - warm), 0.0), 1.0)
    floor = peak * min_ratio
    return floor + (peak - floor) * 0.5 * (1.0 + math.cos(math.pi * prog))


def step(name, step_idx, params, grads, m, v, decay, muon, *, lr, wd=0.1, total=1000,
         warmup=0.02, min_ratio=0.1, b1=0.9, b2=0.95, eps=1e-8, mu=0.95, ns_steps=5,
         cautious_eps=1e-3):
    """One optimizer step; params/grads/m/v: {name: array}; decay, muon: {name: bool}.
    Returns (params, m, v) as new dicts."""
    lr_t = cosine_lr(step_idx, lr, total, warmup, min_ratio)
    t = step_idx + 1.0
    c1, c2 = 1 - b1 ** t, 1 - b2 ** t
    P, Mo, Vo = {}, {}, {}
    for k in params:
        p, g = np.asarray(params[k], F64), np.asarray(grads[k], F64)
        if name in ("muon_adamw", "hybrid_muon_cadamw") and muon[k]:
            mn = mu * m[k] + (1 - mu) * g
            o = newton_schulz_5((1 - mu) * g + mu * mn, steps=ns_steps)
            P[k] = p * (1 - lr_t * wd if decay[k] else 1.0) - lr_t * o
            Mo[k], Vo[k] = mn, None
            continue
        mn = b1 * m[k] + (1 - b1) * g
        vn = b2 * v[k] + (1 - b2) * g * g
        u = (mn / c1) / (np.sqrt(vn / c2) + eps)
        if name in ("cadamw", "hybrid_muon_cadamw"):
            mask = (u * g > 0).astype(F64)
            u = u * (mask / max(mask.mean(), cautious_eps))
        P[k] = p * (1 - lr_t * wd if decay[k] else 1.0) - lr_t * u
        Mo[k], Vo[k] = mn, vn
    return P, Mo, Vo
