"""CPU baseline timing (test/benchmark infrastructure only, never shipped).

Times the reference's dense algebraic attention on the host cores:
``algebraic.asinh_attention`` (src/algebraic/algebraic.py:186-216, with the
max-shifted ``asinh_power_weights``) and its autograd VJP, restated in torch
CPU float32 and evaluated one (b, h) head at a time so the (T, T) score
matrix fits in memory. The reference's own JAX CPU path cannot run here (JAX
is not installed), so this restatement is the timed baseline ("port").
"""

import math
import os
import time

import torch


def _rho(x):
    rad = 1.0 + x * x
    t = x.abs() + rad * torch.rsqrt(rad)
    return torch.where(x >= 0, t, 1.0 / t)


def _ipow(x, n):
    out, base = None, x
    while n:
        if n & 1:
            out = base if out is None else out * base
        n >>= 1
        if n:
            base = base * base
    return out


def dense_asinh_attention(q, k, v, n, c, mask):
    """One head: q, k, v (T, D) float32 -> (T, D), algebraic.py:186-216."""
    d = q.shape[-1]
    s = (q @ k.T) * (1.0 / math.sqrt(d))
    x = s / c
    m = torch.where(mask, x, torch.full_like(x, -1e30)).amax(-1, keepdim=True).detach()
    w = torch.where(mask, _ipow(_rho(x) * _rho(-m), n), torch.zeros_like(x))
    p = w / w.sum(-1, keepdim=True)
    return p @ v


def time_attention_fwd_bwd(T=2048, D=64, n=16, c=8.0, heads=8, threads=None, seed=0):
    """Seconds of each of `heads` single-head forward+backward passes (a
    list), and the thread count."""
    threads = threads or os.cpu_count() or 1
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(seed)
    mask = torch.tril(torch.ones(T, T, dtype=torch.bool))
    times = []
    for _ in range(heads):
        q = torch.randn(T, D, generator=g)
        k = torch.randn(T, D, generator=g)
        q = q * torch.rsqrt((q * q).mean(-1, keepdim=True) + 1e-5)
        k = k * torch.rsqrt((k * k).mean(-1, keepdim=True) + 1e-5)
        v = torch.randn(T, D, generator=g)
        do = torch.randn(T, D, generator=g)
        q.requires_grad_(True)
        k.requires_grad_(True)
        v.requires_grad_(True)
        t0 = time.perf_counter()
        o = dense_asinh_attention(q, k, v, n, c, mask)
        torch.autograd.grad(o, (q, k, v), do)
        times.append(time.perf_counter() - t0)
    return times, threads
