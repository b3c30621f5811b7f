"""GPU parity of qk_rms_norm and fused_head (HIP) against the CPU oracle.

Mirrors tests/test_qk_norm_tpu.py:21-43 and tests/test_fused_head_tpu.py:13-67
of the reference, at the tolerances of tests/_tol.py.
"""

import numpy as np
import pytest
import torch

from _tol import assert_bf16, assert_f32, rel_l2, to_np
from algebraic_amd.kernels import fused_head, qk_rms_norm, qk_rms_norm_pair
from oracle import head as OH
from oracle import qknorm as OQ

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("eps", [1e-5, 1e-3])
@pytest.mark.parametrize("shape", [(2, 3, 512, 64), (8, 16, 2048, 64)])
def test_qk_norm_output_and_vjp(dtype, eps, shape):
    """x = 3 N(0,1) with row 0 zeroed, gain in .25 + 4 U(0,1) (qk_norm TPU test)."""
    rng = np.random.default_rng(181)
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    x = torch.from_numpy((3 * rng.standard_normal(shape)).astype(np.float32)).to(tdt)
    x[0, 0, 0] = 0
    gain = torch.from_numpy((0.25 + 4 * rng.random(64)).astype(np.float32))
    dy = torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(tdt)
    tx = x.to(DEV).requires_grad_(True)
    tg = gain.to(DEV).requires_grad_(True)
    y = qk_rms_norm(tx, tg, eps, block=256)
    (y.float() * dy.to(DEV).float()).sum().backward()
    torch.cuda.synchronize()
    big = shape[0] > 2
    sl = (slice(0, 1), slice(0, 2)) if big else (slice(None),)
    want_y = OQ.forward(to_np(x[sl]), to_np(gain), eps, dtype)
    want_dx, _ = OQ.backward(to_np(x[sl]), to_np(gain), to_np(dy[sl]), eps, dtype)
    check = assert_f32 if dtype == "f32" else assert_bf16
    check(y[sl], want_y, what="y")
    check(tx.grad[sl], want_dx, what="dx")
    if not big:
        _, want_dg = OQ.backward(to_np(x), to_np(gain), to_np(dy), eps, dtype)
        assert rel_l2(tg.grad, want_dg) <= (1e-5 if dtype == "f32" else 1e-3)
    else:
        # dgain over 16.8M rows: compare with a float64 torch reduction on the GPU.
        xf = x.to(DEV).double()
        tau = torch.rsqrt((xf * xf).mean(-1, keepdim=True) + eps)
        dg = (dy.to(DEV).double() * xf * tau).reshape(-1, 64).sum(0)
        assert rel_l2(tg.grad, dg) <= 1e-4


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", [(1, 2, 256, 64), (8, 16, 2048, 64)])
def test_qk_norm_pair_equals_two_calls(dtype, shape):
    """The paired launch returns what two qk_rms_norm calls return, bit for bit
    (y, dx and dgain of q and k), and the q half matches the oracle."""
    rng = np.random.default_rng(563)
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    xs = [torch.from_numpy((2 * rng.standard_normal(shape)).astype(np.float32)).to(tdt)
          for _ in range(2)]
    gs = [torch.from_numpy((1 + 0.01 * rng.standard_normal(64)).astype(np.float32))
          for _ in range(2)]
    dys = [torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(tdt)
           for _ in range(2)]
    ins = [[t.to(DEV).requires_grad_(True) for t in (x, g)] for x, g in zip(xs, gs)]
    single = [qk_rms_norm(x, g, block=256) for x, g in ins]
    torch.autograd.backward(single, [dy.to(DEV) for dy in dys])
    ins2 = [[t.to(DEV).requires_grad_(True) for t in (x, g)] for x, g in zip(xs, gs)]
    pair = qk_rms_norm_pair(ins2[0][0], ins2[1][0], ins2[0][1], ins2[1][1], block=256)
    torch.autograd.backward(pair, [dy.to(DEV) for dy in dys])
    torch.cuda.synchronize()
    for i in range(2):
        assert torch.equal(pair[i], single[i]), f"y[{i}]"
        assert torch.equal(ins2[i][0].grad, ins[i][0].grad), f"dx[{i}]"
        assert torch.equal(ins2[i][1].grad, ins[i][1].grad), f"dgain[{i}]"
    sl = (slice(0, 1), slice(0, 2))
    want = OQ.forward(to_np(xs[0][sl]), to_np(gs[0]), 1e-5, dtype)
    (assert_f32 if dtype == "f32" else assert_bf16)(pair[0][sl], want, what="y_q")


def test_qk_norm_pair_validation():
    q = torch.zeros((2, 4, 64), device=DEV)
    g = torch.ones(64, device=DEV)
    with pytest.raises(ValueError):
        qk_rms_norm_pair(q, torch.zeros((2, 8, 64), device=DEV), g, g, block=8)
    with pytest.raises(ValueError):
        qk_rms_norm_pair(q, q.bfloat16(), g, g, block=8)


def _head_inputs(N, d, V, seed, escale):
    rng = np.random.default_rng(seed)
    h = torch.from_numpy(rng.standard_normal((N, d)).astype(np.float32)).bfloat16()
    e = torch.from_numpy((rng.standard_normal((V, d)) * escale).astype(np.float32))
    t = torch.from_numpy(rng.integers(0, V, N).astype(np.int64))
    return h, e, t


def _head_run(h, e, t, **kw):
    th, te = h.to(DEV).requires_grad_(True), e.to(DEV).requires_grad_(True)
    obj, tel = fused_head(th, te, t.to(DEV), **kw)
    obj.backward()
    torch.cuda.synchronize()
    return float(obj), to_np(tel), to_np(th.grad), to_np(te.grad)


@pytest.mark.parametrize("kind,n,c", [("alg_ce", 16, 16.0), ("alg_ce", 8, 2.0), ("ce", 16, 16.0)])
@pytest.mark.parametrize("V", [4096, 32768, 1000])
def test_fused_head_matches_oracle(kind, n, c, V):
    """N=1024, d=256, E ~ 0.15 N(0,1) (test_fused_head_tpu.py:13-40), plus a ragged V."""
    h, e, t = _head_inputs(1024, 256, V, 0, 0.15)
    got = _head_run(h, e, t, kind=kind, n=n, c=c, block_n=256, block_v=1024)
    (obj, tel), (dh, de) = OH.fused_head(to_np(h), to_np(e), to_np(t), kind=kind, n=n, c=c,
                                         dtype="bf16", g_obj=1.0)
    assert abs(got[0] - obj) <= 2e-4 + 2e-3 * abs(obj)
    np.testing.assert_allclose(got[1], tel, rtol=2e-2, atol=2e-4)
    assert_bf16(got[2], dh, what="dh")
    assert rel_l2(got[3], de) <= 1e-2
    # reference's own check: max-normalised agreement and cosine
    for a, b in ((got[2], dh), (got[3], de)):
        scale = np.abs(b).max() + 1e-12
        np.testing.assert_allclose(a / scale, b / scale, atol=2e-2)
        cos = (a * b).sum() / np.sqrt((a * a).sum() * (b * b).sum())
        assert cos > 0.999


@pytest.mark.parametrize("n", [2, 4, 32, 64, 128])
def test_fused_head_alg_ce_every_unrolled_power(n):
    """alg_ce with the other powers of two: n = 2, 4, 32, 64 run forward
    kernels with compile-time powers, n = 128 the runtime power loop; each
    against the oracle (c = 4, clamp 0.25 (1e38 / V)^(1/n), fused_head.py:273)."""
    h, e, t = _head_inputs(512, 128, 3000, 3, 0.15)
    got = _head_run(h, e, t, kind="alg_ce", n=n, c=4.0)
    (obj, tel), (dh, de) = OH.fused_head(to_np(h), to_np(e), to_np(t), kind="alg_ce", n=n,
                                         c=4.0, dtype="bf16", g_obj=1.0)
    assert abs(got[0] - obj) <= 2e-4 + 2e-3 * abs(obj)
    np.testing.assert_allclose(got[1], tel, rtol=2e-2, atol=2e-4)
    assert_bf16(got[2], dh, what=f"dh n={n}")
    assert rel_l2(got[3], de) <= 1e-2


@pytest.mark.parametrize("N,d,V", [(300, 64, 1000), (600, 40, 257), (8, 128, 300),
                                   (2048, 128, 16284)])
def test_fused_head_ragged_tiles(N, d, V):
    """Token counts and vocabularies that leave partial 256-token and
    vocabulary tiles, and a hidden width that is not a multiple of the 32-wide
    k stage (block_n = N, so the reference's divisibility check holds). The
    last case streams two vocabulary tiles of exactly four k stages per
    workgroup (d = 128) through the direct-to-LDS ring, the last one ragged."""
    h, e, t = _head_inputs(N, d, V, 5, 0.2)
    for kind, n, c in (("alg_ce", 8, 2.0), ("ce", 16, 16.0)):
        got = _head_run(h, e, t, kind=kind, n=n, c=c, block_n=N)
        (obj, tel), (dh, de) = OH.fused_head(to_np(h), to_np(e), to_np(t), kind=kind, n=n, c=c,
                                             dtype="bf16", g_obj=1.0)
        assert abs(got[0] - obj) <= 2e-4 + 2e-3 * abs(obj)
        np.testing.assert_allclose(got[1], tel, rtol=2e-2, atol=2e-4)
        assert_bf16(got[2], dh, what="dh")
        assert rel_l2(got[3], de) <= 1e-2


@pytest.mark.parametrize("kind,n,c", [("alg_ce", 8, 2.0), ("ce", 16, 16.0)])
def test_fused_head_targets_at_tile_and_wave_edges(kind, n, c):
    """The forward and dz kernels test for a target once per wave, token
    column and vocabulary tile (a wave holds 128 rows of a 256-row tile), and
    handle the target logit only where the test holds. Targets here sit on
    both sides of every wave and tile edge, inside the last (partial) tile
    (V = 1000), and 64 consecutive tokens share one target, so whole token
    columns take the target path while their neighbours do not."""
    N, d, V = 512, 64, 1000
    h, e, _ = _head_inputs(N, d, V, 11, 0.2)
    edges = [0, 1, 126, 127, 128, 129, 254, 255, 256, 257, 383, 384, 511, 512,
             767, 768, 895, 896, 997, 998, 999]
    t = np.array([edges[i % len(edges)] for i in range(N)], dtype=np.int64)
    t[128:192] = 200
    t = torch.from_numpy(t)
    got = _head_run(h, e, t, kind=kind, n=n, c=c, block_n=N)
    (obj, tel), (dh, de) = OH.fused_head(to_np(h), to_np(e), to_np(t), kind=kind, n=n, c=c,
                                         dtype="bf16", g_obj=1.0)
    assert abs(got[0] - obj) <= 2e-4 + 2e-3 * abs(obj)
    np.testing.assert_allclose(got[1], tel, rtol=2e-2, atol=2e-4)
    assert_bf16(got[2], dh, what="dh")
    assert rel_l2(got[3], de) <= 1e-2
    # the target rows of E carry the -y r terms: each checked on its own
    rows = sorted(set(edges) | {200})
    assert rel_l2(got[3][rows], de[rows]) <= 1e-2


@pytest.mark.parametrize("width", [768, 1024])
def test_production_head_tiles_at_model_widths(width):
    """test_fused_head_tpu.py:43-67: 256 tokens, V=32768, E ~ 0.02 N(0,1), n=8, c=2."""
    h, e, t = _head_inputs(256, width, 32768, 42, 0.02)
    got = _head_run(h, e, t, kind="alg_ce", n=8, c=2.0)
    (obj, tel), (dh, de) = OH.fused_head(to_np(h), to_np(e), to_np(t), kind="alg_ce", n=8, c=2.0,
                                         dtype="bf16", g_obj=1.0)
    assert abs(got[0] - obj) <= 2e-4 + 2e-3 * abs(obj)
    assert rel_l2(got[2], dh) < 0.01 and rel_l2(got[3], de) < 0.01


@pytest.mark.parametrize("kind,n,c", [("alg_ce", 8, 2.0), ("alg_ce", 16, 16.0), ("ce", 16, 16.0)])
@pytest.mark.parametrize("N,d,V", [(512, 96, 4096), (300, 100, 1000), (64, 768, 50304)])
def test_fused_head_float32_hidden_states(kind, n, c, N, d, V):
    """float32 h: the embedding is cast to float32 and the logits, dz, dh and
    dE are float32 (fused_head.py:160-216 with h.dtype = float32), so the
    outputs meet the float32 tolerance against the float64 oracle. Ragged
    token, vocabulary and width extents (d = 100 is no multiple of 8)."""
    rng = np.random.default_rng(N + d)
    h = torch.from_numpy(rng.standard_normal((N, d)).astype(np.float32))
    e = torch.from_numpy((rng.standard_normal((V, d)) * 0.15).astype(np.float32))
    t = torch.from_numpy(rng.integers(0, V, N).astype(np.int64))
    got = _head_run(h, e, t, kind=kind, n=n, c=c, block_n=N)
    (obj, tel), (dh, de) = OH.fused_head(to_np(h), to_np(e), to_np(t), kind=kind, n=n, c=c,
                                         dtype="f32", g_obj=1.0)
    assert abs(got[0] - obj) <= 1e-5 * abs(obj) + 1e-7
    assert_f32(got[1], tel, what="telemetry")
    assert_f32(got[2], dh, what="dh")
    assert_f32(got[3], de, what="dE")


def test_fused_head_alg_gradient_is_log_loss_gradient():
    """The alg_ce VJP equals the exact NLL gradient of log_softmax(n asinh(z/c))."""
    h, e, t = _head_inputs(256, 128, 4096, 9, 0.3)
    got = _head_run(h, e, t, kind="alg_ce", n=8, c=2.0)
    th = torch.tensor(to_np(h), requires_grad=True)
    te = torch.tensor(to_np(e.bfloat16()), requires_grad=True)
    z = th @ te.T
    logp = torch.log_softmax(8 * torch.asinh(z / 2.0), -1)[torch.arange(256), t]
    (-logp.mean()).backward()
    assert rel_l2(got[2], th.grad.numpy()) < 1e-2
    assert rel_l2(got[3], te.grad.numpy()) < 1e-2
    np.testing.assert_allclose(got[1], np.exp(logp.detach().numpy()), rtol=2e-2, atol=2e-6)


def test_fused_head_backward_over_token_chunks(monkeypatch):
    """With the bf16 logit-gradient scratch capped at 512 MiB, N=12288 tokens at
    V=50304 run as three token chunks, the later ones accumulating dE.
    Checked against dense float32 math on the GPU: the
    objective mean(1 - p_t) (algebraic.py:243-245) and, as the reference's
    custom VJP returns, the gradient of the mean NLL of
    log_softmax(n asinh(z/c)) (the clamp is inactive at these logits)."""
    monkeypatch.setenv("ALGX_HEAD_CHUNK_BYTES", str(512 << 20))
    N, d, V, n, c = 12288, 64, 50304, 8, 2.0
    gen = torch.Generator(device=DEV).manual_seed(7)
    h = torch.randn((N, d), device=DEV, generator=gen).bfloat16()
    e = (0.02 * torch.randn((V, d), device=DEV, generator=gen)).bfloat16()
    t = torch.randint(0, V, (N,), device=DEV, generator=gen)
    th, te = h.clone().requires_grad_(True), e.clone().requires_grad_(True)
    obj, _ = fused_head(th, te, t, kind="alg_ce", n=n, c=c)
    obj.backward()
    rh, re = h.float().requires_grad_(True), e.float().requires_grad_(True)
    logp = torch.log_softmax(n * torch.asinh((rh @ re.T) / c), -1).gather(1, t[:, None])
    ref = float((1.0 - logp.detach().exp()).mean())
    (-logp.mean()).backward()
    torch.cuda.synchronize()
    assert abs(float(obj) - ref) <= 2e-4 + 2e-3 * abs(ref)
    assert rel_l2(th.grad, rh.grad) <= 1e-2
    assert rel_l2(te.grad, re.grad) <= 1e-2
    for a, b in ((th.grad, rh.grad), (te.grad, re.grad)):
        assert float((a.float() - b).abs().max()) <= 2e-2 * float(b.abs().max())


@pytest.mark.parametrize("kind,n,c", [("alg_ce", 8, 2.0), ("ce", 16, 16.0)])
def test_fused_head_at_benchmark_shape(kind, n, c):
    """configs[2] exactly: N=16384 tokens, d=768, V=50304 (one 1.65 GB dz chunk,
    a ragged last 256-row vocabulary tile), h ~ N(0,1), E ~ 0.02 N(0,1), bf16.
    Checked against dense float32 math on the GPU: objective, telemetry p_t,
    and the gradients of the mean NLL of log_softmax(n asinh(z/c)) (alg_ce) or
    of the cross entropy (ce), which are the reference's custom VJPs."""
    N, d, V = 16384, 768, 50304
    gen = torch.Generator(device=DEV).manual_seed(2)
    h = torch.randn((N, d), device=DEV, generator=gen).bfloat16()
    e = (0.02 * torch.randn((V, d), device=DEV, generator=gen)).bfloat16()
    t = torch.randint(0, V, (N,), device=DEV, generator=gen)
    th, te = h.clone().requires_grad_(True), e.clone().requires_grad_(True)
    obj, tel = fused_head(th, te, t, kind=kind, n=n, c=c)
    obj.backward()
    rh, re = h.float().requires_grad_(True), e.float().requires_grad_(True)
    z = rh @ re.T
    logits = n * torch.asinh(z / c) if kind == "alg_ce" else z
    logp = torch.log_softmax(logits, -1).gather(1, t[:, None])[:, 0]
    lp = logp.detach()
    ref_obj = float((1.0 - lp.exp()).mean()) if kind == "alg_ce" else float(-lp.mean())
    (-logp.mean()).backward()
    torch.cuda.synchronize()
    assert abs(float(obj) - ref_obj) <= 2e-4 + 2e-3 * abs(ref_obj)
    # telemetry: p_t for alg_ce, the per-token NLL for ce (fused_head.py:219-229)
    want_tel = logp.exp() if kind == "alg_ce" else -logp
    np.testing.assert_allclose(to_np(tel), to_np(want_tel.detach()), rtol=2e-2, atol=2e-6)
    assert rel_l2(th.grad, rh.grad) <= 1e-2
    assert rel_l2(te.grad, re.grad) <= 1e-2
    # Elementwise: the gradients are O(1/N), so the bf16 bar's 2e-2 is taken
    # relative to each tensor's largest entry (max |a - b| <= 2e-2 max |b|).
    for a, b in ((th.grad, rh.grad), (te.grad, re.grad)):
        assert float((a.float() - b).abs().max()) <= 2e-2 * float(b.abs().max())
