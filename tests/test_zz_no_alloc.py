"""algx_attn_forward_noalloc against algx_attn_forward (C ABI, GPU).

The no-allocation entry point keeps the range guard's partial maxima in the
library's per-device scratch array instead of a caller workspace; its
outputs must equal the workspace entry point's bit for bit. Two calls in a
row (the second on a smaller input, so the scratch holds the first call's
larger contents) and both guard outcomes (in range, and the out-of-range
tail that makes the fallback kernel read the partials).
"""

import math

import numpy as np
import pytest
import torch

from algebraic_amd import _lib
from algebraic_amd.kernels.flash import _c_variant, make_variant

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(shape, seed, tail):
    rng = np.random.default_rng(seed)
    q, k, v = (torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).bfloat16().to(DEV)
               for _ in range(3))
    if tail:
        q = torch.full_like(q, math.sqrt(1000.0))
        k = q.clone()
    return q, k, v


def _forward(q, k, v, sink, noalloc):
    """One guarded n=16, c=8 forward (flash.py:834-856's pair); returns the
    outputs and the guard word."""
    B, H, T, D = q.shape
    var = make_variant("asinh", 16, 8.0, seq_len=T)
    low = var._replace(shift=False, inv_stat=True, bounded_scores=True)
    high = var._replace(shift=True, inv_stat=False, fast_rho=False, bounded_scores=False,
                        head_resident=False, precise_output=True)
    lo, hi = _c_variant(low), _c_variant(high)
    bound = min(16.0, var.clamp / 2)
    q_scale = 1.0 / (8.0 * math.sqrt(D))
    vmax = min(1e8, 1e37 / ((T + 1) * (2 * bound + 1) ** 16))
    guard = torch.zeros(_lib.query("algx_attn_guard_words"), dtype=torch.int32, device=DEV)
    q_s, o = torch.empty_like(q), torch.empty_like(q)
    stat = torch.empty((B, H, T), dtype=torch.float32, device=DEV)
    o_precise = torch.zeros(q.shape, dtype=torch.float32, device=DEV)
    # The backward workspace the forward prepares: its dQ accumulator (the
    # first B*H*T*D floats) starts as NaN and must come back zero.
    bws = torch.full((_lib.query("algx_attn_bwd_workspace_bytes", B, H, T, D) // 4,),
                     float("nan"), dtype=torch.float32, device=DEV)
    common = (_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(sink), _lib.ptr(q_s), _lib.ptr(o),
              _lib.ptr(o_precise), _lib.ptr(stat), _lib.ptr(guard))
    tail = (B, H, T, D, _lib.BF16, q_scale, bound, vmax, lo, hi, _lib.stream())
    if noalloc:
        _lib.call("algx_attn_forward_noalloc", *common, _lib.ptr(bws), *tail)
    else:
        ws = torch.empty(_lib.query("algx_attn_forward_workspace_bytes", B, H, T, D),
                         dtype=torch.uint8, device=DEV)
        _lib.call("algx_attn_forward", *common, _lib.ptr(ws), _lib.ptr(bws), *tail)
    torch.cuda.synchronize()
    return int(guard[0].item()), q_s, o, stat, o_precise, bws[: B * H * T * D]


@pytest.mark.parametrize("tail", [False, True])
def test_noalloc_forward_equals_workspace_forward(tail):
    sink3 = torch.tensor([0.25, -0.5, 0.0], device=DEV)
    for shape, seed in (((2, 3, 1024, 64), 5), ((1, 2, 256, 64), 6)):
        q, k, v = _inputs(shape, seed, tail)
        sink = sink3[: shape[1]].contiguous()
        want = _forward(q, k, v, sink, noalloc=False)
        got = _forward(q, k, v, sink, noalloc=True)
        assert got[0] == want[0] == (0 if tail else 1), (shape, got[0], want[0])
        for a, b, name in zip(got[1:], want[1:], ("q_s", "o", "stat", "o_precise", "dq_acc")):
            assert torch.equal(a, b), (shape, name)
        assert not got[5].any(), shape
