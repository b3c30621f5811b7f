"""GPU parity of flash_attention (HIP) against the CPU oracle.

Mirrors the reference's TPU suite (tests/test_flash_kernel_tpu.py): the
variant cases of test_flash_matches_dense, the model statistics modes, the
guarded tails, the clip VJP, and the whole-head model shape; plus
size-independent properties at the benchmark shape (cfg2/cfg4: B=8, T=2048).
Tolerances: tests/_tol.py (float32 rtol 1e-4; bf16 2e-2 max-abs, 1e-2 rel-L2).
"""

import math
import os

import numpy as np
import pytest
import torch

from _tol import assert_bf16, assert_dtype_close, assert_f32, rel_l2, to_np
from algebraic_amd import _lib
from algebraic_amd.kernels import flash_attention
from oracle import attention as OA

pytestmark = pytest.mark.gpu
DEV = "cuda"
TORCH_DT = {"bf16": torch.bfloat16, "f32": torch.float32}


def _rand(shape, seed, scale=1.0, dtype="bf16", n=4):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        x = torch.from_numpy((rng.standard_normal(shape) * scale).astype(np.float32))
        out.append(x.to(TORCH_DT[dtype]))
    return out


def _run(q, k, v, g, sink, **kw):
    """Forward + VJP on the GPU; returns numpy (o, dq, dk, dv, dsink)."""
    tq, tk, tv = (x.to(DEV).requires_grad_(True) for x in (q, k, v))
    ts = None if sink is None else torch.as_tensor(sink, dtype=torch.float32, device=DEV).requires_grad_(True)
    o = flash_attention(tq, tk, tv, ts, **kw)
    (o.float() * g.to(DEV).float()).sum().backward()
    torch.cuda.synchronize()
    return (to_np(o), to_np(tq.grad), to_np(tk.grad), to_np(tv.grad),
            None if ts is None else to_np(ts.grad))


def _oracle(q, k, v, g, sink, dtype, **kw):
    res = OA.flash_attention(to_np(q), to_np(k), to_np(v), None if sink is None else to_np(sink),
                             dtype=dtype, do=to_np(g), **kw)
    return (res.o,) + tuple(res.grads), res


def _check_all(got, want, dtype, names=("o", "dq", "dk", "dv", "dsink")):
    for a, b, nm in zip(got, want, names):
        if a is None and b is None:
            continue
        if nm == "dsink":
            # float32 reduction over B*T rows in both implementations.
            assert rel_l2(a, b) <= (1e-4 if dtype == "f32" else 1e-2), (nm, a, b)
            continue
        assert_dtype_close(a, b, dtype, what=nm)


def test_mfma_lane_layout_selftest():
    """One v_mfma_f32_32x32x16_bf16 with the layout all MFMA kernels assume."""
    rng = np.random.default_rng(0)
    a = torch.from_numpy(rng.standard_normal((32, 16)).astype(np.float32)).to(torch.bfloat16)
    bt = torch.from_numpy(rng.standard_normal((32, 16)).astype(np.float32)).to(torch.bfloat16)
    d = torch.empty((32, 32), dtype=torch.float32, device=DEV)
    ad, btd = a.to(DEV), bt.to(DEV)
    _lib.call("algx_selftest_mfma32", _lib.ptr(ad), _lib.ptr(btd), _lib.ptr(d), _lib.stream())
    torch.cuda.synchronize()
    want = a.double().numpy() @ bt.double().numpy().T
    np.testing.assert_allclose(d.cpu().numpy(), want, rtol=1e-5, atol=1e-5)


# test_flash_kernel_tpu.py:33-35 plus the model preset and the softmax arm
CASES = [("asinh", 16, 16.0, True, True, False), ("asinh", 16, 16.0, True, True, True),
         ("asinh", 16, 16.0, True, False, True), ("asinh", 16, 16.0, False, False, True),
         ("asinh", 8, 1.0, True, True, False), ("asinh", 32, 8.0, False, True, True),
         ("softmax", 16, 16.0, True, None, None), ("softmax", 16, 16.0, False, None, None)]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("kind,n,c,with_sink,shift,fast", CASES)
def test_flash_matches_oracle(kind, n, c, with_sink, shift, fast, dtype):
    """Every explicit variant, both dtypes, B,H,T,D = 2,3,256,64, inputs x1.5."""
    shape = (2, 3, 256, 64)
    q, k, v, g = _rand(shape, 0, dtype=dtype)
    q, k = ((x.float() * 1.5).to(TORCH_DT[dtype]) for x in (q, k))
    sink = (torch.from_numpy(np.random.default_rng(4).standard_normal(3).astype(np.float32)) * 0.5
            ).reshape(1, 3, 1, 1) if with_sink else None
    kw = dict(kind=kind, n=n, c=c, shift=shift, fast_rho=fast)
    got = _run(q, k, v, g, sink, block=128, **kw)
    want, res = _oracle(q, k, v, g, sink, dtype, **kw)
    _check_all(got, want, dtype)


@pytest.mark.parametrize("n", [2, 4, 64])
@pytest.mark.parametrize("shift", [False, True])
def test_mfma_runtime_power(n, shift):
    """bf16 MFMA kernels with n outside 8..32, whose weight takes its n-th
    power in a runtime loop (the kernels built for three workgroups per CU),
    forward and backward against the oracle, with a sink."""
    shape = (1, 2, 256, 64)
    q, k, v, g = _rand(shape, 40 + n + int(shift))
    sink = torch.tensor([0.4, -0.3]).reshape(1, 2, 1, 1)
    kw = dict(kind="asinh", n=n, c=8.0, shift=shift)
    got = _run(q, k, v, g, sink, block=128, **kw)
    want, _ = _oracle(q, k, v, g, sink, "bf16", **kw)
    _check_all(got, want, "bf16")


@pytest.mark.parametrize("T", [128, 384])
@pytest.mark.parametrize("kw", [dict(kind="asinh", n=16, c=8.0, range_guard=True),
                                dict(kind="asinh", n=16, c=16.0, shift=True, fast_rho=True),
                                dict(kind="softmax")], ids=["guarded", "shift", "softmax"])
def test_mfma_forward_block_counts(T, kw):
    """bf16 MFMA kernels at one 128-query block (only the two diagonal key
    tiles, no unmasked loop) and at an odd block count (the backward's last
    256-key block half empty), against the oracle."""
    shape = (1, 2, T, 64)
    q, k, v, g = _rand(shape, 11 + T)
    sink = (torch.tensor([0.3, -0.7]).reshape(1, 2, 1, 1)
            if kw["kind"] == "softmax" else None)
    got = _run(q, k, v, g, sink, block=128, **kw)
    want, _ = _oracle(q, k, v, g, sink, "bf16", **kw)
    _check_all(got, want, "bf16")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("mode", ["root", "inverse", "guarded"])
def test_model_attention_statistics(mode, dtype):
    """test_flash_kernel_tpu.py:69-97: n=16, c=8 with a sink, statistic modes."""
    shape = (1, 2, 512, 64)
    q, k, v, g = _rand(shape, 13, dtype=dtype)
    sink = torch.from_numpy(np.random.default_rng(14).standard_normal((1, 2, 1, 1)).astype(np.float32))
    kw = dict(kind="asinh", n=16, c=8.0, shift=False, fast_rho=True, inv_stat=mode != "root",
              range_guard=mode == "guarded")
    got = _run(q, k, v, g, sink, block_q=128, block_k=256, **kw)
    want, res = _oracle(q, k, v, g, sink, dtype, **kw)
    if mode == "guarded":
        assert res.in_range
    _check_all(got, want, dtype)
    # the reference's own check against the dense function (0.012 / rel 0.02|0.005)
    dense = OA.dense_asinh_attention(to_np(q), to_np(k), to_np(v), n=16, c=8.0, sink_logit=to_np(sink),
                                     p_dtype=dtype)
    np.testing.assert_allclose(got[0], dense, atol=0.012, rtol=0.012)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("score_sign", [-1.0, 1.0])
@pytest.mark.parametrize("with_sink", [False, True])
@pytest.mark.parametrize("magnitude", [1000.0, 1e7])
def test_guarded_attention_tail(score_sign, with_sink, magnitude, dtype):
    """test_flash_kernel_tpu.py:100-119: guarded fallback for overflow and underflow."""
    shape = (1, 1, 256, 64)
    q = torch.full(shape, math.sqrt(magnitude), dtype=TORCH_DT[dtype])
    k = (q.float() * score_sign).to(TORCH_DT[dtype])
    v = _rand(shape, 29, dtype=dtype, n=1)[0]
    g = torch.ones(shape, dtype=TORCH_DT[dtype])
    sink = torch.zeros((1,)) if with_sink else None
    kw = dict(kind="asinh", n=16, c=8.0, range_guard=True)
    got = _run(q, k, v, g, sink, block=128, **kw)
    want, res = _oracle(q, k, v, g, sink, dtype, **kw)
    assert res.in_range is False
    assert all(np.isfinite(x).all() for x in got[:4])
    dense = OA.dense_asinh_attention(to_np(q), to_np(k), to_np(v), n=16, c=8.0,
                                     sink_logit=None if sink is None else to_np(sink), p_dtype=dtype)
    tol = 2e-3 if dtype == "f32" else 0.012
    np.testing.assert_allclose(got[0], dense, atol=tol, rtol=tol)
    assert_dtype_close(got[0], want[0], dtype, what="o")


def test_explicit_clipping_vjp_is_zero_above_cap():
    """test_flash_kernel_tpu.py:122-138: saturated scores and sink have zero VJP."""
    shape = (1, 1, 256, 64)
    q = torch.full(shape, math.sqrt(1000), dtype=torch.float32)
    v, g = _rand(shape, 39, dtype="f32", n=2)
    got = _run(q, q.clone(), v, g, torch.full((1,), 1000.0), kind="asinh", n=16, c=8.0,
               block=128, shift=False, range_guard=False)
    for x in (got[1], got[2], got[4]):
        assert np.all(x == 0)


@pytest.mark.parametrize("mode", ["sink", "no_sink", "negative", "gain_two", "positive_tail",
                                  "negative_tail"])
def test_whole_head_model_shape(mode):
    """test_flash_kernel_tpu.py:253-328 at (1, 2, 2048, 64) bf16, guarded n=16, c=8."""
    shape = (1, 2, 2048, 64)
    q, k, v, g = _rand(shape, 563)
    sink = torch.tensor([-0.35, 0.125]).reshape(1, 2, 1, 1)
    if mode in ("no_sink", "negative"):
        sink = None
    if mode == "negative":
        q = (1 + 0.05 * q.float()).to(torch.bfloat16)
        k = (-1 + 0.05 * k.float()).to(torch.bfloat16)
    if mode == "gain_two":
        q = (2 * q.float() * torch.rsqrt((q.float() ** 2).mean(-1, keepdim=True) + 1e-5)).to(torch.bfloat16)
        k = (2 * k.float() * torch.rsqrt((k.float() ** 2).mean(-1, keepdim=True) + 1e-5)).to(torch.bfloat16)
    if mode.endswith("tail"):
        q = torch.full(shape, math.sqrt(1000), dtype=torch.bfloat16)
        k = q if mode == "positive_tail" else (-q.float()).to(torch.bfloat16)
    kw = dict(kind="asinh", n=16, c=8.0, range_guard=True)
    got = _run(q, k, v, g, sink, **kw)
    want, res = _oracle(q, k, v, g, sink, "bf16", **kw)
    assert res.in_range == (not mode.endswith("tail"))
    names = ("o", "dq", "dk", "dv", "dsink")
    for a, b, nm in zip(got, want, names):
        if a is None:
            continue
        if nm == "dq" and mode in ("positive_tail", "negative"):
            # Equal or nearly common scores make dQ a small difference of bf16-rounded
            # terms (test_flash_kernel_tpu.py:205-207, :295-314): absolute check only.
            assert np.abs(a - b).max() <= 2e-2, (mode, np.abs(a - b).max())
            continue
        if nm == "dsink":
            assert rel_l2(a, b) <= 1e-2
            continue
        assert_bf16(a, b, what=f"{mode}:{nm}")


@pytest.mark.parametrize("qscale", [1.0, 3.0])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("blocks", [(128, 128), (128, 256), (256, 128)])
def test_model_attention_polynomial_radical(dtype, blocks, qscale):
    """test_flash_kernel_tpu.py:69-97, mode "polynomial": poly_rho (the
    bounded radical, radical.py:26-38) at n=16, c=8 with a sink against the
    exact functions with the reference's tolerances; and against the oracle's
    restatement of the reference's per-tile choice, within the polynomial's
    approximation error (the kernels choose per score). qscale 3 puts the
    largest |x| near 2, so score tiles cross |x| = 1 and the per-score and
    per-tile choices differ."""
    shape = (1, 2, 512, 64)
    q, k, v, g = _rand(shape, 13, dtype=dtype)
    if qscale != 1.0:
        q = (q.float() * qscale).to(q.dtype)
    sink = torch.from_numpy(np.random.default_rng(14).standard_normal((1, 2, 1, 1)).astype(np.float32))
    kw = dict(kind="asinh", n=16, c=8.0, shift=False, fast_rho=True, inv_stat=True)
    bq, bk = blocks
    got = _run(q, k, v, g, sink, block_q=bq, block_k=bk, poly_rho=True, **kw)
    dense = OA.dense_asinh_attention(to_np(q), to_np(k), to_np(v), n=16, c=8.0, sink_logit=to_np(sink),
                                     p_dtype=dtype)
    np.testing.assert_allclose(got[0], dense, atol=0.012, rtol=0.012)
    exact, _ = _oracle(q, k, v, g, sink, dtype, kind="asinh", n=16, c=8.0, shift=False,
                       fast_rho=False, inv_stat=True)
    for a, b in zip(got[1:], exact[1:]):
        assert rel_l2(a, b) < (0.02 if dtype == "bf16" else 0.005)
    poly, _ = _oracle(q, k, v, g, sink, dtype, poly_rho=True, block_q=bq, block_k=bk, **kw)
    for a, b, nm in zip(got, poly, ("o", "dq", "dk", "dv", "dsink")):
        if dtype == "f32":
            # weights differ by at most the polynomial's error (~7e-4 at n=16)
            assert rel_l2(a, b) <= 2e-3, (nm, rel_l2(a, b))
        elif nm == "dsink":
            assert rel_l2(a, b) <= 1e-2, (nm, rel_l2(a, b))
        else:
            assert_dtype_close(a, b, dtype, what=nm)


def test_polynomial_radical_refuses_guard_and_shift():
    q = torch.zeros((1, 1, 64, 64), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="range_guard"):
        flash_attention(q, q, q, kind="asinh", n=16, c=8.0, poly_rho=True, range_guard=True,
                        shift=False)
    with pytest.raises(ValueError, match="shift=False and n=16"):
        flash_attention(q, q, q, kind="asinh", n=16, c=8.0, poly_rho=True, shift=True)


def test_mfma_path_matches_generic_kernels():
    """The MFMA kernels and the scalar kernels agree on every output (bf16, T=512)."""
    shape = (2, 4, 512, 64)
    q, k, v, g = _rand(shape, 77)
    sink = torch.tensor([0.3, -0.2, 0.0, 1.0]).reshape(1, 4, 1, 1)
    kw = dict(kind="asinh", n=16, c=8.0, range_guard=True)
    fast = _run(q, k, v, g, sink, **kw)
    os.environ["ALGX_FORCE_GENERIC"] = "1"
    try:
        slow = _run(q, k, v, g, sink, **kw)
    finally:
        del os.environ["ALGX_FORCE_GENERIC"]
    for a, b, nm in zip(fast, slow, ("o", "dq", "dk", "dv", "dsink")):
        assert rel_l2(a, b) <= 5e-3, (nm, rel_l2(a, b))


@pytest.mark.parametrize("H", [12, 16])
def test_benchmark_shape_properties(H):
    """cfg2/cfg4 shape (8, H, 2048, 64) bf16, QK-normed inputs, guarded n=16, c=8:
    the in-range path runs; outputs are finite; weights sum to one (v = 1 gives
    o = 1); the output is causal (perturbing later keys leaves earlier rows
    unchanged); and one head matches the oracle."""
    B, T, D = 8, 2048, 64
    shape = (B, H, T, D)
    gen = torch.Generator(device=DEV).manual_seed(1)
    q = torch.randn(shape, device=DEV, generator=gen)
    k = torch.randn(shape, device=DEV, generator=gen)
    q = (q * torch.rsqrt((q * q).mean(-1, keepdim=True) + 1e-5)).bfloat16()
    k = (k * torch.rsqrt((k * k).mean(-1, keepdim=True) + 1e-5)).bfloat16()
    v = torch.randn(shape, device=DEV, generator=gen).bfloat16()
    kw = dict(kind="asinh", n=16, c=8.0, range_guard=True)
    o = flash_attention(q, k, v, **kw)
    assert torch.isfinite(o.float()).all()
    ones = flash_attention(q, k, torch.ones_like(v), **kw).float()
    assert (ones - 1).abs().max().item() <= 8e-3
    k2 = k.clone()
    k2[:, :, 1024:] = (k2[:, :, 1024:].float() * -3).bfloat16()
    o2 = flash_attention(q, k2, v, **kw)
    assert torch.equal(o[:, :, :1024], o2[:, :, :1024])
    # one head against the oracle
    qs, ks, vs = (x[3:4, 5:6].cpu() for x in (q, k, v))
    res = OA.flash_attention(to_np(qs), to_np(ks), to_np(vs), None, dtype="bf16", **kw)
    assert res.in_range
    assert_bf16(o[3:4, 5:6], res.o, what="o(head)")


@pytest.mark.parametrize("tail", [False, True])
def test_fused_forward_equals_prepare_then_forward(tail):
    """algx_attn_forward (pre-scale and guard fused into the MFMA forward, high
    variant behind the guard word) gives the same q_s, o, stat and guard
    decision as algx_attn_prepare followed by algx_attn_fwd."""
    from algebraic_amd.kernels.flash import _c_variant, make_variant

    B, H, T, D = 2, 3, 512, 64
    q, k, v = (x.to(DEV) for x in _rand((B, H, T, D), 91, n=3))
    if tail:
        q = torch.full_like(q, math.sqrt(1000.0))
        k = q.clone()
    sink = torch.tensor([0.25, -0.5, 0.0], device=DEV)
    # The guarded pair flash_attention builds for n=16, c=8 (flash.py:834-856).
    var = make_variant("asinh", 16, 8.0, seq_len=T)
    low = var._replace(shift=False, inv_stat=True, bounded_scores=True)
    high = var._replace(shift=True, inv_stat=False, fast_rho=False, bounded_scores=False,
                        head_resident=False, precise_output=True)
    lo, hi = _c_variant(low), _c_variant(high)
    bound = min(16.0, var.clamp / 2)
    q_scale, vmax = 1.0 / (8.0 * math.sqrt(D)), min(1e8, 1e37 / ((T + 1) * (2 * bound + 1) ** 16))
    st = _lib.stream()
    words = _lib.query("algx_attn_guard_words")
    outs = []
    for fused in (True, False):
        guard = torch.zeros(words, dtype=torch.int32, device=DEV)
        q_s, o = torch.empty_like(q), torch.empty_like(q)
        stat = torch.empty((B, H, T), dtype=torch.float32, device=DEV)
        o_precise = torch.empty(q.shape, dtype=torch.float32, device=DEV)
        if fused:
            ws = torch.empty(_lib.query("algx_attn_forward_workspace_bytes", B, H, T, D),
                             dtype=torch.uint8, device=DEV)
            _lib.call("algx_attn_forward", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(sink),
                      _lib.ptr(q_s), _lib.ptr(o), _lib.ptr(o_precise), _lib.ptr(stat),
                      _lib.ptr(guard), _lib.ptr(ws), None, B, H, T, D,
                      _lib.dtype_code(q.dtype), q_scale, bound, vmax, lo, hi, st)
        else:
            _lib.call("algx_attn_prepare", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(sink),
                      _lib.ptr(q_s), _lib.ptr(guard), B, H, T, D, _lib.dtype_code(q.dtype),
                      q_scale, bound, vmax, st)
            _lib.call("algx_attn_fwd", _lib.ptr(q_s), _lib.ptr(k), _lib.ptr(v), _lib.ptr(sink),
                      _lib.ptr(o), _lib.ptr(o_precise), _lib.ptr(stat), B, H, T, D,
                      _lib.dtype_code(q.dtype), lo, hi, _lib.ptr(guard), st)
        torch.cuda.synchronize()
        outs.append((int(guard[0].item()), q_s, o, stat))
    (g1, qs1, o1, s1), (g2, qs2, o2, s2) = outs
    assert g1 == g2 == (0 if tail else 1)
    assert torch.equal(qs1, qs2)
    assert torch.equal(o1, o2)
    assert torch.equal(s1, s2)


# Heads with a nonzero output gradient in the full-grid backward test: their
# b*H + h fall on XCD slots 3, 5 and 7 (b*H + h mod 8) at H = 12 and H = 16.
_GRAD_HEADS = ((0, 3), (2, 5), (6, 7))


@pytest.mark.parametrize("with_sink", [False, True])
@pytest.mark.parametrize("H", [12, 16])
def test_benchmark_shape_backward_selected_heads(H, with_sink):
    """The whole (8, H, 2048, 64) bf16 guarded grid runs forward and backward
    (768 or 1024 backward workgroups, the float32 dQ atomics, the XCD head
    map), with dO nonzero in three heads on different XCD slots: those heads'
    o, dq, dk, dv (and, with a per-head sink, dsink) match the oracle and
    every other head's gradients are exactly zero. Without a sink and with dO
    dense instead, sum_keys dV = sum_queries dO for every (b, h, d) (the
    weights of each query row sum to one)."""
    B, T, D = 8, 2048, 64
    shape = (B, H, T, D)
    gen = torch.Generator(device=DEV).manual_seed(11)
    q = torch.randn(shape, device=DEV, generator=gen)
    k = torch.randn(shape, device=DEV, generator=gen)
    q = (q * torch.rsqrt((q * q).mean(-1, keepdim=True) + 1e-5)).bfloat16()
    k = (k * torch.rsqrt((k * k).mean(-1, keepdim=True) + 1e-5)).bfloat16()
    v = torch.randn(shape, device=DEV, generator=gen).bfloat16()
    do_full = torch.randn(shape, device=DEV, generator=gen).bfloat16()
    do = torch.zeros_like(do_full)
    heads = list(_GRAD_HEADS)
    assert sorted((b * H + h) % 8 for b, h in heads) == [3, 5, 7]
    for b, h in heads:
        do[b, h] = do_full[b, h]
    kw = dict(kind="asinh", n=16, c=8.0, range_guard=True)
    tq, tk, tv = (x.clone().requires_grad_(True) for x in (q, k, v))
    ts = None
    if with_sink:
        ts = (0.5 * torch.randn(H, device=DEV, generator=gen)).requires_grad_(True)
    o = flash_attention(tq, tk, tv, ts, **kw)
    grads = torch.autograd.grad(o, (tq, tk, tv) + ((ts,) if with_sink else ()), do)
    dq, dk, dv = grads[:3]
    torch.cuda.synchronize()
    mask = torch.ones((B, H), dtype=torch.bool)
    for b, h in heads:
        mask[b, h] = False
    for name, g in (("dq", dq), ("dk", dk), ("dv", dv)):
        assert torch.count_nonzero(g[mask.to(DEV)]) == 0, name
    if with_sink:
        dsink = to_np(grads[3])
        others = [h for h in range(H) if h not in {hh for _, hh in heads}]
        assert np.count_nonzero(dsink[others]) == 0
    for b, h in heads:
        sl = (slice(b, b + 1), slice(h, h + 1))
        res = OA.flash_attention(to_np(q[sl]), to_np(k[sl]), to_np(v[sl]),
                                 to_np(ts[h:h + 1]) if with_sink else None, dtype="bf16",
                                 do=to_np(do[sl]), **kw)
        assert res.in_range
        assert_bf16(o[sl], res.o, what=f"o{b, h}")
        for got, want, name in zip((dq, dk, dv), res.grads[:3], ("dq", "dk", "dv")):
            assert_bf16(got[sl], want, what=f"{name}{b, h}")
        if with_sink:
            assert rel_l2(dsink[h:h + 1], res.grads[3]) <= 1e-2, (h, dsink[h], res.grads[3])
    if with_sink:
        return
    # dense dO: column sums of dV equal those of dO, head by head
    dv_full = torch.autograd.grad(flash_attention(tq, tk, tv, **kw), tv, do_full)[0]
    lhs = dv_full.double().sum(2)
    rhs = do_full.double().sum(2)
    err = (lhs - rhs).abs().max().item()
    assert err <= 2e-2 * rhs.abs().max().item() + 0.5, err
    assert rel_l2(lhs, rhs) <= 5e-3


def test_guarded_tail_at_benchmark_shape():
    """Out-of-range inputs at (8, 12, 2048, 64): 1536 query tiles go through
    the high-variant fallback grid of 512 workgroups, so each workgroup walks
    three tiles (the grid-stride loop). One head against the oracle."""
    B, H, T, D = 8, 12, 2048, 64
    shape = (B, H, T, D)
    q = torch.full(shape, math.sqrt(1000.0), dtype=torch.bfloat16, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(12)
    v = torch.randn(shape, device=DEV, generator=gen).bfloat16()
    do = torch.randn(shape, device=DEV, generator=gen).bfloat16()
    kw = dict(kind="asinh", n=16, c=8.0, range_guard=True)
    tq, tk, tv = (x.clone().requires_grad_(True) for x in (q, q, v))
    o = flash_attention(tq, tk, tv, **kw)
    dq, dk, dv = torch.autograd.grad(o, (tq, tk, tv), do)
    torch.cuda.synchronize()
    assert all(torch.isfinite(x.float()).all() for x in (o, dq, dk, dv))
    for b, h in ((0, 0), (5, 7), (7, 11)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        res = OA.flash_attention(to_np(q[sl]), to_np(q[sl]), to_np(v[sl]), None, dtype="bf16",
                                 do=to_np(do[sl]), **kw)
        assert res.in_range is False
        assert_bf16(o[sl], res.o, what=f"o{b, h}")
        assert_bf16(dv[sl], res.grads[2], what=f"dv{b, h}")
        # equal scores: dq, dk are differences of nearly equal bf16-rounded
        # terms (test_flash_kernel_tpu.py:205-207): absolute check only
        for got, want in ((dq, res.grads[0]), (dk, res.grads[1])):
            assert np.abs(to_np(got[sl]) - want).max() <= 2e-2


def test_bf16_clipping_vjp_is_zero_above_cap():
    """test_flash_kernel_tpu.py:122-138 in bf16 through the MFMA kernels: every
    score (and the sink) above the unguarded clamp of shift=False, n=16, T=256
    (72.58) has a zero VJP."""
    shape = (1, 1, 256, 64)
    q = torch.full(shape, math.sqrt(1000), dtype=torch.bfloat16)
    v, g = _rand(shape, 39, n=2)
    got = _run(q, q.clone(), v, g, torch.full((1,), 1000.0), kind="asinh", n=16, c=8.0,
               block=128, shift=False, range_guard=False)
    for x in (got[1], got[2], got[4]):
        assert np.all(x == 0)
    assert np.isfinite(got[0]).all() and np.isfinite(got[3]).all()


@pytest.mark.parametrize("with_sink", [False, True])
def test_bf16_partly_clipped_scores_match_oracle(with_sink):
    """bf16, shift=False, unguarded, T=256: q, k ~ 20 N(0,1) puts a share of
    the scores above the clamp (72.58) and the rest below it, so the MFMA
    backward's clamp kink (zero score gradient at and above the clamp) and
    the clamped weights meet ordinary ones in the same tiles."""
    shape = (2, 2, 256, 64)
    q, k, v, g = _rand(shape, 41)
    q, k = ((x.float() * 20).bfloat16() for x in (q, k))
    qs = q.float() / 64.0
    s = qs @ k.float().transpose(-1, -2)
    frac = (s > 72.58).float().tril().sum() / torch.ones_like(s).tril().sum()
    assert 0.01 < frac.item() < 0.5, frac.item()
    sink = torch.tensor([0.5, 1000.0]).reshape(1, 2, 1, 1) if with_sink else None
    kw = dict(kind="asinh", n=16, c=8.0, shift=False, range_guard=False)
    got = _run(q, k, v, g, sink, block=128, **kw)
    want, _ = _oracle(q, k, v, g, sink, "bf16", **kw)
    for a, b, nm in zip(got, want, ("o", "dq", "dk", "dv", "dsink")):
        if a is None:
            continue
        if nm == "dsink":
            assert np.abs(a - b).max() <= 1e-2 * max(1.0, np.abs(b).max()), (a, b)
            continue
        assert_bf16(a, b, what=nm)


@pytest.mark.parametrize("kind,shift", [("asinh", False), ("asinh", True), ("softmax", True)])
def test_precise_output_in_every_mode(kind, shift):
    """A C-ABI caller may ask for the float32 output with any variant: the MFMA
    forward writes o_precise in every mode (o is its bf16 rounding), and the
    backward's di read from it gives the gradients of the bf16 residual to
    within bf16 accuracy."""
    from algebraic_amd.kernels.flash import _c_variant, make_variant

    B, H, T, D = 1, 2, 256, 64
    q, k, v, do = (x.to(DEV) for x in _rand((B, H, T, D), 93, n=4))
    var = make_variant(kind, 16, 8.0, seq_len=T)
    if kind == "asinh":
        var = var._replace(shift=shift, inv_stat=not shift, bounded_scores=not shift)
    st = _lib.stream()
    outs = []
    for precise in (1, 0):
        lo = _c_variant(var._replace(precise_output=bool(precise)))
        q_s = (q.float() * (1.0 / (8.0 * math.sqrt(D)) if kind == "asinh" else
                            1.0 / math.sqrt(D))).bfloat16()
        o = torch.empty_like(q)
        o_precise = torch.full(q.shape, float("nan"), dtype=torch.float32, device=DEV)
        stat = torch.empty((B, H, T), dtype=torch.float32, device=DEV)
        _lib.call("algx_attn_fwd", _lib.ptr(q_s), _lib.ptr(k), _lib.ptr(v), None, _lib.ptr(o),
                  _lib.ptr(o_precise), _lib.ptr(stat), B, H, T, D, _lib.BF16, lo, None, None, st)
        dq, dk, dv = (torch.empty_like(q) for _ in range(3))
        ws = torch.empty(_lib.query("algx_attn_bwd_workspace_bytes", B, H, T, D),
                         dtype=torch.uint8, device=DEV)
        _lib.call("algx_attn_bwd", _lib.ptr(q_s), _lib.ptr(k), _lib.ptr(v), None, _lib.ptr(o),
                  _lib.ptr(o_precise), _lib.ptr(stat), _lib.ptr(do), _lib.ptr(dq), _lib.ptr(dk),
                  _lib.ptr(dv), None, _lib.ptr(ws), _lib.ATTN_WS_RAW, B, H, T, D, _lib.BF16, 1.0,
                  lo, None, None, st)
        torch.cuda.synchronize()
        if precise:
            assert torch.isfinite(o_precise).all()
            assert torch.equal(o_precise.bfloat16(), o)
        outs.append((dq, dk, dv))
    for a, b in zip(*outs):
        assert torch.isfinite(a.float()).all()
        assert rel_l2(a, b) <= 5e-3


@pytest.mark.parametrize("kind", ["asinh", "softmax"])
def test_prepared_workspace_backward_matches_raw(kind):
    """flash_attention's backward runs on the workspace its forward prepared
    (ALGX_ATTN_WS_CLEARED: the forward cleared the dQ accumulator, the
    backward's pre-pass only forms di). A second backward of the same graph
    (retain_graph) gets a raw workspace, which the pre-pass clears. Both
    match the oracle; dk and dv agree bit for bit (dq sums float32 atomics in
    an order that may vary from run to run)."""
    B, H, T, D = 2, 3, 512, 64
    q, k, v, g = _rand((B, H, T, D), 97)
    kw = (dict(kind="asinh", n=16, c=8.0, range_guard=True) if kind == "asinh"
          else dict(kind="softmax"))
    tq, tk, tv = (x.to(DEV).requires_grad_(True) for x in (q, k, v))
    o = flash_attention(tq, tk, tv, None, **kw)
    gd = g.to(DEV)
    first = torch.autograd.grad(o, (tq, tk, tv), gd, retain_graph=True)
    second = torch.autograd.grad(o, (tq, tk, tv), gd)
    torch.cuda.synchronize()
    (_, *want), _ = _oracle(q, k, v, g, None, "bf16", **kw)
    for got in (first, second):
        for a, b, nm in zip(got, want, ("dq", "dk", "dv")):
            assert_bf16(to_np(a), b, what=nm)
    assert torch.equal(first[1], second[1]) and torch.equal(first[2], second[2])
    assert rel_l2(first[0], second[0]) <= 1e-3
