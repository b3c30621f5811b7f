"""The model over the HIP operators against the float64 model oracle (GPU).

A small model of each preset (2 layers, 2 heads of 32 or 64 -- the latter
through the fused attention prologue --, d_ff 96, V = 97, T = 16; weights at init_std 0.1 with perturbed gains and sink logits
so every path carries signal) runs one forward + backward; its objective,
telemetry and every parameter gradient are compared with torch float64
autograd of ``oracle.model`` on the same parameters and tokens.

* float32 with the dense head: each operator computes in float32, so the
  model agrees with float64 to float32 accuracy: relative L2 <= 1e-4 per
  gradient tensor (the north star's float32 rtol).
* bfloat16 with the fused head (the configuration the model trains in): the
  activations are rounded to bf16 after every operator (~2^-9 relative each)
  across two blocks, and the gradients pass through the same roundings
  backwards; the bar is relative L2 <= 3e-2 per gradient tensor and 1e-2 on
  the objective -- an integration bar, above the per-operator ones (1e-2
  relative L2) which every operator meets in its own tests.

Plus the 350M algebraic preset at its real width for one sequence of 2048
tokens and V = 50304 (finite objective and gradients, the MFMA paths); both
350M presets at configs[4]'s full size (B = 8 x 2048) through a whole
training step, with the final head checked against dense float32 math; and
rematerialisation against no rematerialisation.
"""

import math

import numpy as np
import pytest
import torch

from _tol import rel_l2, to_np
from algebraic_amd import config, model
from algebraic_amd.kernels import fused_head
from oracle import model as OM

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cfg(preset, dtype, head_impl, head_dim=32, **kw):
    # head_dim 64 takes the fused attention prologue, 32 the operators one by one
    return config.build(preset, "proxy", d_model=2 * head_dim, n_layers=2, n_heads=2, d_ff=96,
                        vocab_size=97, seq_len=16, init_std=0.1, dtype=dtype,
                        head_impl=head_impl, attn_impl="flash", **kw)


def _perturb(params, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    with torch.no_grad():
        for name in ("embed_gain", "final_gain"):
            if name in params:
                params[name].add_(0.2 * torch.randn(params[name].shape, generator=g, device=DEV))
        for name in ("ln1", "ln2", "q_gain", "k_gain"):
            if name in params["layers"]:
                t = params["layers"][name]
                t.add_(0.2 * torch.randn(t.shape, generator=g, device=DEV))
        if "sink" in params["layers"]:
            t = params["layers"]["sink"]
            t.copy_(torch.randn(t.shape, generator=g, device=DEV))


def _flat(tree, prefix=""):
    out = {}
    for k, v in tree.items():
        if isinstance(v, dict):
            out.update(_flat(v, prefix + k + "."))
        else:
            out[prefix + k] = v
    return out


def _to_f64(tree):
    return {k: _to_f64(v) if isinstance(v, dict) else
            v.detach().cpu().to(torch.float64).requires_grad_(True) for k, v in tree.items()}


def _run(cfg, seed=0):
    params = model.init_params(cfg, seed=seed, device=DEV)
    _perturb(params, seed + 1)
    g = torch.Generator(device=DEV).manual_seed(seed + 2)
    tok = torch.randint(0, cfg.vocab_size, (2, 16), generator=g, device=DEV)
    tgt = torch.randint(0, cfg.vocab_size, (2, 16), generator=g, device=DEV)
    tables = model.position_tables(cfg, 16, device=DEV)
    obj, tel = model.train_objective(params, tok, tgt, cfg, tables)
    obj.backward()
    torch.cuda.synchronize()
    ref = _to_f64(params)
    r_obj, r_tel, r_loss = OM.forward(ref, tok.cpu(), tgt.cpu(), cfg)
    r_loss.backward()
    return params, obj, tel, ref, r_obj, r_tel


@pytest.mark.parametrize("head_dim", [32, 64])
@pytest.mark.parametrize("preset", ["algebraic", "standard"])
@pytest.mark.parametrize("dtype,head_impl,grad_tol,obj_tol", [
    ("float32", "dense", 1e-4, 1e-5),
    ("float32", "fused", 1e-4, 1e-5),
    ("bfloat16", "fused", 3e-2, 1e-2),
])
def test_small_model_matches_oracle(preset, dtype, head_impl, grad_tol, obj_tol, head_dim):
    cfg = _cfg(preset, dtype, head_impl, head_dim)
    params, obj, tel, ref, r_obj, r_tel = _run(cfg)
    assert abs(float(obj.detach()) - float(r_obj.detach())) <= obj_tol * abs(float(r_obj.detach()))
    assert rel_l2(tel, r_tel) <= obj_tol * 10
    got, want = _flat(params), _flat(ref)
    assert set(got) == set(want)
    for name in sorted(got):
        gg, ww = got[name].grad, want[name].grad
        assert gg is not None, name
        err = rel_l2(gg, ww)
        assert err <= grad_tol, f"{name}: gradient rel-L2 {err:.2e} > {grad_tol}"


def test_remat_matches_no_remat():
    """Recomputing each block in the backward gives the gradients of storing it."""
    grads = []
    for remat in (True, False):
        cfg = _cfg("algebraic", "bfloat16", "fused", remat=remat)
        params, *_ = _run(cfg, seed=5)
        grads.append({k: v.grad.clone() for k, v in _flat(params).items()})
    for name in grads[0]:
        assert rel_l2(grads[0][name], grads[1][name]) <= 1e-3, name


def test_350m_algebraic_step_is_finite():
    """One fwd + bwd of the 350M algebraic preset (d 1024, 24 layers, 16 heads
    of 64, d_ff 2688) on one 2048-token sequence with V = 50304."""
    cfg = config.algebraic("350m", vocab_size=50304, seq_len=2048, attn_impl="flash",
                           head_impl="fused")
    params = model.init_params(cfg, seed=0, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(1)
    tok = torch.randint(0, 50304, (1, 2048), generator=g, device=DEV)
    tables = model.position_tables(cfg, device=DEV)
    obj, tel = model.train_objective(params, tok[:, :], torch.roll(tok, -1, 1), cfg, tables)
    obj.backward()
    torch.cuda.synchronize()
    assert torch.isfinite(obj) and torch.isfinite(tel).all()
    # mean(1 - p_t) with p_t ~ 1/V at init: just below one
    assert 0.99 < float(obj.detach()) <= 1 and 0 < float(tel.min()) and float(tel.max()) < 0.01
    for name, t in _flat(params).items():
        assert t.grad is not None and torch.isfinite(t.grad).all(), name
    assert float(params["layers"]["w_q"].grad.abs().max()) > 0


def _dense_head_slice(h, E, t, cfg, n_total):
    """Dense float32 head on one slice of tokens (h (M, d) bf16, E (V, d)):
    the objective's gradients w.r.t. h and E scaled as the slice's part of a
    mean over n_total tokens. alg_ce differentiates the exact NLL of
    log_softmax(n asinh(z/c)) (the reference's custom VJP,
    algebraic.py:255-262), ce the cross entropy (standard.py:41-47)."""
    rh = h.detach().float().requires_grad_(True)
    re = E.detach().to(torch.bfloat16).float().requires_grad_(True)
    z = rh @ re.T
    logits = cfg.head_n * torch.asinh(z / cfg.head_c) if cfg.head == "alg_ce" else z
    logp = torch.log_softmax(logits, -1).gather(1, t[:, None].long())[:, 0]
    (-logp.sum() / n_total).backward()
    return rh.grad, re.grad, logp.detach()


@pytest.mark.parametrize("preset", ["algebraic", "standard"])
def test_350m_training_step_at_benchmark_shape(preset):
    """configs[4] at its stated size: the 350M preset (d 1024, 24 layers, 16
    heads of 64, d_ff 2688, V 50304; model.py:196-231, config.py:17-42) on
    B = 8 x T = 2048 random tokens, no rematerialisation, forward + backward
    and one Muon + AdamW step (optimizers.py:118-246).

    * the objective and the per-token telemetry against dense float32 math
      on the model's final hidden states (mean(1 - p_t) just below one for
      alg_ce at init; for ce the tied embedding puts each position's own
      input token far ahead, so the cross entropy sits above ln V);
    * every gradient finite and not all zero; every parameter finite and
      changed by the step;
    * the final head on the model's own last hidden states: the model's dh
      for the first sequence (2048 tokens) against dense float32 math of that
      slice's part of the mean, and the fused head called on that slice
      alone (dh and dE) against the same dense math."""
    from algebraic_amd import optimizers
    B, T, V = 8, 2048, 50304
    cfg = config.build(preset, "350m", vocab_size=V, seq_len=T, attn_impl="flash",
                       head_impl="fused", remat=False)
    params = model.init_params(cfg, seed=0, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(5)
    tok = torch.randint(0, V, (B, T + 1), generator=g, device=DEV)
    x, y = tok[:, :-1].contiguous(), tok[:, 1:].contiguous()
    tables = model.position_tables(cfg, T, device=DEV)
    hidden = model.forward_hidden(params, x, cfg, tables)
    hidden.retain_grad()
    obj, tel = model.head_loss(params, hidden, y, cfg)
    obj.backward()
    torch.cuda.synchronize()
    o = float(obj.detach())
    assert math.isfinite(o) and torch.isfinite(tel).all()
    # the objective and telemetry against dense float32 math over all B T
    # tokens (2048 at a time)
    E16 = params["embed"].detach().to(torch.bfloat16).float()
    hs, ys = hidden.detach().reshape(B * T, -1), y.reshape(B * T)
    lps = []
    with torch.no_grad():
        for i in range(0, B * T, T):
            z = hs[i:i + T].float() @ E16.T
            logits = cfg.head_n * torch.asinh(z / cfg.head_c) if cfg.head == "alg_ce" else z
            lps.append(torch.log_softmax(logits, -1).gather(1, ys[i:i + T, None].long())[:, 0])
    lp = torch.cat(lps)
    del E16, lps
    ref_obj = float((1.0 - lp.exp()).mean()) if cfg.head == "alg_ce" else float(-lp.mean())
    assert abs(o - ref_obj) <= 2e-4 + 2e-3 * abs(ref_obj), (o, ref_obj)
    want_tel = lp.exp() if cfg.head == "alg_ce" else -lp
    np.testing.assert_allclose(to_np(tel), to_np(want_tel), rtol=2e-2, atol=2e-6)
    if cfg.head == "alg_ce":
        # mean(1 - p_t) with p_t far below one at init: just below one
        assert 0.99 < o <= 1.0, o
    flat = _flat(params)
    for name, t in flat.items():
        assert t.grad is not None and torch.isfinite(t.grad).all(), name
        assert bool((t.grad != 0).any()), f"{name}: gradient is all zero"

    # the head on the model's own final hidden states, first sequence
    h0, t0 = hidden[0].detach(), y[0]
    dh_ref, de_ref, logp = _dense_head_slice(h0, params["embed"], t0, cfg, B * T)
    assert rel_l2(hidden.grad[0], dh_ref) <= 1e-2
    th = h0.clone().requires_grad_(True)
    te = params["embed"].detach().to(torch.bfloat16).requires_grad_(True)
    s_obj, s_tel = fused_head(th, te, t0, kind=cfg.head, n=cfg.head_n, c=cfg.head_c)
    s_obj.backward()
    torch.cuda.synchronize()
    want_tel = logp.exp() if cfg.head == "alg_ce" else -logp
    np.testing.assert_allclose(to_np(s_tel), to_np(want_tel), rtol=2e-2, atol=2e-6)
    # the slice alone averages over T tokens, the reference over B * T
    assert rel_l2(th.grad.float() / B, dh_ref) <= 1e-2
    assert rel_l2(te.grad.float() / B, de_ref) <= 1e-2
    del dh_ref, de_ref, th, te

    init_fn, step_fn = optimizers.get_optimizer("muon_adamw", 2e-3, weight_decay=0.1,
                                                total_steps=100, warmup_fraction=0.0)
    state = init_fn(params)
    before = {k: v.detach().clone() for k, v in flat.items()}
    step_fn(0, params, optimizers.grads_of(params), state, model.decay_mask(params))
    torch.cuda.synchronize()
    for name, t in _flat(params).items():
        assert torch.isfinite(t).all(), name
        assert not torch.equal(t.detach(), before[name]), f"{name}: unchanged by the step"
    del params, before, state, hidden, flat
    torch.cuda.empty_cache()


@pytest.mark.parametrize("preset", ["algebraic", "standard"])
def test_training_reduces_the_loss(preset):
    """Twenty Muon + AdamW steps on one fixed batch of a small model (the
    reference trainer's default optimizer): the true log loss (from the
    telemetry) falls well below its starting value, and every parameter
    stays finite."""
    import math
    from algebraic_amd import optimizers
    cfg = config.build(preset, "proxy", d_model=128, n_layers=2, n_heads=2, d_ff=96,
                       vocab_size=97, seq_len=32, attn_impl="flash", head_impl="fused",
                       remat=False)
    params = model.init_params(cfg, seed=7, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(8)
    tok = torch.randint(0, 97, (4, 33), generator=g, device=DEV)
    x, y = tok[:, :-1].contiguous(), tok[:, 1:].contiguous()
    tables = model.position_tables(cfg, 32, device=DEV)
    init_fn, step_fn = optimizers.get_optimizer("muon_adamw", 2e-2, total_steps=20,
                                                warmup_fraction=0.1)
    state = init_fn(params)
    mask = model.decay_mask(params)
    nll = []
    for s in range(20):
        for t in _flat(params).values():
            t.grad = None
        obj, tel = model.train_objective(params, x, y, cfg, tables)
        obj.backward()
        nll.append(float((-tel.log()).mean()) if model.telemetry_is_probability(cfg)
                   else float(tel.mean()))
        step_fn(s, params, optimizers.grads_of(params), state, mask)
    torch.cuda.synchronize()
    assert all(math.isfinite(v) for v in nll)
    assert nll[-1] < 0.7 * nll[0], nll
    for name, t in _flat(params).items():
        assert torch.isfinite(t).all(), name
