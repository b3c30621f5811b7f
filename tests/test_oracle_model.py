"""Pins for the float64 model oracle and the host-side model pieces (no GPU).

``oracle.model`` restates the reference Transformer from textbook formulas;
these tests check its parts against what shares none of its code: complex
powers for the Cayley tables (and the reference's own closed-form check of
the float32 tables, test_components.py:59-68), the other attention and head
restatements of ``oracle/`` (pinned in tests/test_oracle.py), causality, and
the reference's parameter count for the 350M preset.
"""

import numpy as np
import pytest
import torch

from algebraic_amd import config, model
from oracle import attention as OA
from oracle import head as OH
from oracle import model as OM


def test_cayley_tables_are_complex_powers():
    """cos/sin(m phi), phi = 2 atan w, equal ((1 + i w)^2 / (1 + w^2))^m."""
    half, T = 16, 300
    w = 0.5 * 1e4 ** (-np.arange(half) / half)
    z = (1 + 1j * w) ** 2 / (1 + w * w)
    zm = z[None, :] ** np.arange(T)[:, None]
    c, s = OM.tables("cayley_geo", 2 * half, T)
    np.testing.assert_allclose(c.numpy(), zm.real, atol=1e-12)
    np.testing.assert_allclose(s.numpy(), zm.imag, atol=1e-12)


def test_model_tables_match_closed_forms():
    """test_components.py:59-68 (atol 2e-5) for the float32 binary powering;
    RoPE against cos/sin of m theta; partial rotary keeps w = 0 frequencies fixed."""
    c, s = model.cayley_table_geometric(64, 300, device="cpu")
    m = np.arange(300)[:, None]
    ang = 2 * np.arctan(0.5 * 1e4 ** (-np.arange(32) / 32))
    np.testing.assert_allclose(c.numpy(), np.cos(m * ang), atol=2e-5)
    np.testing.assert_allclose(s.numpy(), np.sin(m * ang), atol=2e-5)
    np.testing.assert_allclose(c.numpy() ** 2 + s.numpy() ** 2, 1.0, atol=1e-6)
    oc, os_ = OM.tables("cayley_geo", 64, 300)
    np.testing.assert_allclose(c.numpy(), oc.numpy(), atol=2e-5)
    np.testing.assert_allclose(s.numpy(), os_.numpy(), atol=2e-5)
    rc, rs = model.rope_table(64, 300, device="cpu")
    orc, ors = OM.tables("rope", 64, 300)
    np.testing.assert_allclose(rc.numpy(), orc.numpy(), atol=2e-4)
    np.testing.assert_allclose(rs.numpy(), ors.numpy(), atol=2e-4)
    pc, ps = model.cayley_table_geometric(64, 50, fraction=0.5, device="cpu")
    assert torch.all(pc[:, 16:] == 1) and torch.all(ps[:, 16:] == 0)
    c16, s16 = model.cayley_table_geometric(16, 4, device="cpu")   # test_e2e_requirements.py:1018-1024
    assert torch.isfinite(c16).all() and torch.isfinite(s16).all()


@pytest.mark.parametrize("kind,n,c", [("asinh", 16, 8.0), ("softmax", 16, 1.0)])
@pytest.mark.parametrize("with_sink", [False, True])
def test_oracle_attention_matches_other_restatement(kind, n, c, with_sink):
    rng = np.random.default_rng(3)
    q, k, v = (rng.standard_normal((2, 3, 9, 8)) for _ in range(3))
    sink = rng.standard_normal(3) if with_sink else None
    got = OM.attention(*(torch.tensor(x) for x in (q, k, v)),
                       None if sink is None else torch.tensor(sink), kind, n, c)
    if kind == "asinh":
        want = OA.dense_asinh_attention(q, k, v, n=n, c=c, sink_logit=sink)
    else:
        want = OA.dense_softmax_attention(q, k, v, sink_logit=sink)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-10, atol=1e-12)


def _tiny(preset, **kw):
    return config.build(preset, "proxy", d_model=32, n_layers=1, n_heads=2, d_ff=24,
                        vocab_size=41, seq_len=8, **kw)


def _f64(params):
    def conv(t):
        return {k: conv(v) for k, v in t.items()} if isinstance(t, dict) else \
            t.detach().to(torch.float64).requires_grad_(True)
    return conv(params)


@pytest.mark.parametrize("preset", ["algebraic", "standard"])
def test_oracle_identity_blocks_reduce_to_the_head(preset):
    """With w_o = w_d = 0 every block is the identity, so the objective and
    telemetry are the head oracle's on rms(rms(embed[tokens]))."""
    cfg = _tiny(preset)
    p = _f64(model.init_params(cfg, seed=1, device="cpu"))
    with torch.no_grad():
        p["layers"]["w_o"].zero_()
        p["layers"]["w_d"].zero_()
        p["embed_gain"].uniform_(0.5, 1.5)
        p["final_gain"].uniform_(0.5, 1.5)
    tok = torch.randint(0, 41, (2, 8), generator=torch.Generator().manual_seed(2))
    obj, tel, _ = OM.forward(p, tok, tok, cfg)
    e = p["embed"].detach()
    x = e[tok]
    for g in (p["embed_gain"], p["final_gain"]):
        x = x / torch.sqrt((x * x).mean(-1, keepdim=True) + cfg.eps) * g.detach()
    kw = dict(kind=cfg.head, n=cfg.head_n, c=cfg.head_c, dtype="f64", embed_dtype="f64")
    (want_obj, want_tel), _ = OH.fused_head(x.reshape(16, 32).numpy(), e.numpy(),
                                            tok.reshape(-1).numpy(), **kw)
    assert float(obj.detach()) == pytest.approx(want_obj, rel=1e-10)
    np.testing.assert_allclose(tel.numpy(), want_tel, rtol=1e-9)


@pytest.mark.parametrize("preset", ["algebraic", "standard"])
def test_oracle_is_causal(preset):
    """Changing the last token changes no telemetry at earlier positions."""
    cfg = _tiny(preset)
    p = _f64(model.init_params(cfg, seed=3, device="cpu"))
    tok = torch.randint(0, 41, (1, 8), generator=torch.Generator().manual_seed(4))
    tok2 = tok.clone()
    tok2[0, -1] = (tok[0, -1] + 1) % 41
    _, t1, _ = OM.forward(p, tok, tok, cfg)
    _, t2, _ = OM.forward(p, tok2, tok, cfg)
    np.testing.assert_allclose(t1[:-1].numpy(), t2[:-1].numpy(), rtol=1e-12)
    assert t1[-1] != t2[-1]


def test_presets_and_parameter_count():
    """config.py:8-49; 'both arms have approximately 332.45M parameters' with
    the tied 32k embedding (config.py:12)."""
    a, s = config.algebraic("350m"), config.standard("350m")
    assert a.algebraic_path and not s.algebraic_path
    assert (a.ffn, a.alu_beta, a.pos, a.attn, a.attn_n, a.attn_c, a.sink, a.head, a.head_n,
            a.head_c, a.qk_norm) == ("alu_glu", 0.5, "cayley_geo", "asinh", 16, 8.0, "learned",
                                     "alg_ce", 8, 2.0, True)
    assert (s.ffn, s.pos, s.attn, s.head) == ("swiglu", "rope", "softmax", "ce")
    L, d, f, V, H = 24, 1024, 2688, 32768, 16
    dense = V * d + L * (4 * d * d + 3 * d * f)
    n_std = dense + 2 * d + 2 * L * d
    n_alg = n_std + 2 * L * 64 + L * H
    assert abs(n_std / 1e6 - 332.45) < 0.05 and abs(n_alg / 1e6 - 332.45) < 0.05
    small = config.algebraic("proxy", d_model=64, n_layers=2, n_heads=2, d_ff=96, vocab_size=97)
    p = model.init_params(small, device="cpu")
    want = 97 * 64 + 2 * (4 * 64 * 64 + 3 * 64 * 96) + 2 * 64 + 2 * 2 * 64 + 2 * 2 * 32 + 2 * 2
    assert model.count_params(p) == want
    assert model.decay_mask(p)["layers"]["w_q"] and not model.decay_mask(p)["layers"]["ln1"]


def test_prologue_oracle_rotation_is_complex_multiplication_and_vjp_is_autograd():
    """Rotate-half = (x1 + i x2) e^{i phi}; the whole chain's VJP equals torch
    float64 autograd of norm -> rotation -> transpose."""
    from oracle import prologue as OP
    rng = np.random.default_rng(9)
    B, T, H, D = 2, 5, 3, 64
    x = rng.standard_normal((B, T, H, D)) * 2
    gain = 0.5 + rng.random(D)
    phi = rng.random((T, D // 2)) * 6
    cos, sin = np.cos(phi), np.sin(phi)
    got = OP.forward(x, None, cos, sin, 1e-5, "f64")
    z = (x[..., :32] + 1j * x[..., 32:]) * np.exp(1j * phi)[None, :, None, :]
    np.testing.assert_allclose(got, np.transpose(np.concatenate([z.real, z.imag], -1),
                                                 (0, 2, 1, 3)), atol=1e-12)
    dout = rng.standard_normal((B, H, T, D))
    tx = torch.tensor(x, requires_grad=True)
    tg = torch.tensor(gain, requires_grad=True)
    y = tx / torch.sqrt((tx * tx).mean(-1, keepdim=True) + 1e-5) * tg
    c, s = torch.tensor(cos)[None, :, None, :], torch.tensor(sin)[None, :, None, :]
    y = torch.cat([y[..., :32] * c - y[..., 32:] * s, y[..., :32] * s + y[..., 32:] * c], -1)
    out = y.transpose(1, 2)
    (out * torch.tensor(dout)).sum().backward()
    np.testing.assert_allclose(OP.forward(x, gain, cos, sin, 1e-5, "f64"),
                               out.detach().numpy(), rtol=1e-12, atol=1e-12)
    dx, dg = OP.backward(x, gain, cos, sin, dout, 1e-5, "f64")
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dg, tg.grad.numpy(), rtol=1e-6)
