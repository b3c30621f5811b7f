"""Pins the function bench.py times as its CPU baseline.

``oracle.cpu_baseline.dense_asinh_attention`` (torch CPU float32, the
reference's dense algebraic.asinh_attention, algebraic.py:186-216) and its
autograd VJP are compared with the float64 oracle, whose forward and closed
VJP are pinned against textbook softmax, float64 autograd and finite
differences in test_oracle.py. Agreement to float32 accuracy shows the timed
baseline computes the same attention (a dropped shift, a wrong scale or a
missing mask would fail it).
"""

import math

import numpy as np
import pytest
import torch

from _tol import rel_l2
from oracle import attention as OA
from oracle.cpu_baseline import dense_asinh_attention, time_attention_fwd_bwd


@pytest.mark.parametrize("T,scale,seed", [(64, 1.0, 0), (128, 1.0, 1), (128, 6.0, 2)])
def test_cpu_baseline_matches_oracle(T, scale, seed):
    """One head, n=16, c=8 (the bench's variant). scale=6 puts scores far from
    zero (|s/c| up to ~20), where the running-max shift matters."""
    D, n, c = 64, 16, 8.0
    rng = np.random.default_rng(seed)
    q, k, v, do = (rng.standard_normal((T, D)) for _ in range(4))
    q, k = q * scale, k * scale
    tq, tk, tv = (torch.tensor(x, dtype=torch.float32, requires_grad=True) for x in (q, k, v))
    mask = torch.tril(torch.ones(T, T, dtype=torch.bool))
    o = dense_asinh_attention(tq, tk, tv, n, c, mask)
    dq, dk, dv = torch.autograd.grad(o, (tq, tk, tv), torch.tensor(do, dtype=torch.float32))
    as4 = lambda x: np.asarray(x, np.float32).astype(np.float64)[None, None]
    res = OA.flash_attention(as4(q), as4(k), as4(v), None, kind="asinh", n=n, c=c, dtype="f64",
                             do=as4(do))
    assert rel_l2(o.detach().numpy(), res.o[0, 0]) <= 1e-5
    for got, want, name in zip((dq, dk, dv), res.grads[:3], ("dq", "dk", "dv")):
        assert rel_l2(got.numpy(), want[0, 0]) <= 1e-4, name


def test_cpu_baseline_timer_runs():
    """The timing helper returns one positive time per head and the thread count."""
    times, threads = time_attention_fwd_bwd(T=128, D=64, heads=2, threads=1)
    assert len(times) == 2 and all(t > 0 for t in times) and threads == 1
    assert math.isfinite(sum(times))
