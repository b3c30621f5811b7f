"""CPU oracle: the reference Transformer in textbook float64 (test infrastructure only).

Restates src/algebraic/model.py:162-231 with formulas that share no code with
the HIP operators or with ``algebraic_amd.model``:

* rms_norm as x / sqrt(mean(x^2) + eps) * gain (algebraic.py:76-83);
* rotations from closed-form angles: RoPE cos(m theta_k) (standard.py:16-21);
  the geometric Cayley grid as cos(m phi_k), sin(m phi_k) with
  phi_k = 2 atan(w_k), w_k = 1/2 base^(-k/half) -- the angle of
  (1 + i w)^2 / (1 + w^2) (algebraic.py:124-169, and the reference's own
  check test_components.py:59-68);
* asinh attention as softmax over the compressed logits n asinh(s/c) with the
  sink as one more logit n asinh(sink/c) (the identity of
  test_components.py:28-41); softmax attention with the raw sink logit
  (standard.py:24-38);
* ALU by its closed form, SwiGLU as up * sigmoid(up) * gate;
* heads: "ce" mean(logsumexp - z_t) (standard.py:41-47); "alg_ce" with
  p = softmax(n asinh(min(z/c, X))), objective mean(1 - p_t), telemetry p_t,
  and as the differentiated loss mean(-log p_t), whose gradient is the
  reference's custom VJP (n/c) r (p - y) / N (algebraic.py:232-262, 286-320;
  test_components.py:44-56).

``grad_loss`` is what torch autograd differentiates to give the reference's
parameter gradients; for "ce" it equals the objective.
"""

import math

import torch

F64 = torch.float64


def _rms_norm(x, gain, eps):
    y = x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps)
    return y * gain if gain is not None else y


def tables(pos, head_dim, T, base=10000.0, fraction=1.0):
    """(cos, sin) of shape (T, head_dim/2) from closed-form angles."""
    half = head_dim // 2
    m = torch.arange(T, dtype=F64)[:, None]
    if pos == "rope":
        theta = 1.0 / (base ** (torch.arange(half, dtype=F64) / half))
        ang = m * theta[None, :]
    elif pos == "cayley_geo":
        active = int(round(fraction * half))
        w = torch.tensor([0.5 * base ** (-k / half) if k < active else 0.0 for k in range(half)],
                         dtype=F64)
        ang = m * (2.0 * torch.atan(w))[None, :]
    elif pos == "none":
        ang = torch.zeros((T, half), dtype=F64)
    else:
        raise ValueError(pos)
    return torch.cos(ang), torch.sin(ang)


def _rotate(x, cos, sin):
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], -1)


def attention(q, k, v, sink, kind, n, c):
    """Dense causal attention on (B, H, T, D); sink: (H,) logits or None."""
    B, H, T, D = q.shape
    s = q @ k.transpose(-1, -2) / math.sqrt(D)
    if kind == "asinh":
        logits = n * torch.asinh(s / c)
    else:
        logits = s
    mask = torch.tril(torch.ones((T, T), dtype=torch.bool))
    logits = logits.masked_fill(~mask, float("-inf"))
    if sink is not None:
        sl = n * torch.asinh(sink / c) if kind == "asinh" else sink
        col = sl.reshape(1, H, 1, 1).expand(B, H, T, 1)
        p = torch.softmax(torch.cat([logits, col], -1), -1)[..., :-1]
    else:
        p = torch.softmax(logits, -1)
    return p @ v


def _alu(x, beta):
    return 0.5 * x * (1 + beta * x / torch.sqrt(1 + (beta * x) ** 2))


def _lean_clamp(vocab, n):
    return 0.25 * (1e38 / vocab) ** (1.0 / n)


def forward(params, tokens, targets, cfg):
    """(objective, telemetry, grad_loss) of model.py:194-231 in float64.

    ``params``: the model's parameter tree as float64 CPU tensors (leaves may
    require grad); ``cfg``: an LMConfig-like object."""
    B, T = tokens.shape
    H, D, d = cfg.n_heads, cfg.d_model // cfg.n_heads, cfg.d_model
    rms = cfg.norm == "rms"
    cos, sin = tables(cfg.pos, D, T, cfg.rope_base, cfg.rope_fraction)
    x = params["embed"][tokens]
    x = _rms_norm(x, params["embed_gain"] if rms else None, cfg.eps)
    lay = params["layers"]
    for i in range(cfg.n_layers):
        h = _rms_norm(x, lay["ln1"][i] if rms else None, cfg.eps)
        q = (h @ lay["w_q"][i]).reshape(B, T, H, D).transpose(1, 2)
        k = (h @ lay["w_k"][i]).reshape(B, T, H, D).transpose(1, 2)
        v = (h @ lay["w_v"][i]).reshape(B, T, H, D).transpose(1, 2)
        if cfg.qk_norm:
            q = _rms_norm(q, lay["q_gain"][i], cfg.eps)
            k = _rms_norm(k, lay["k_gain"][i], cfg.eps)
        q, k = _rotate(q, cos, sin), _rotate(k, cos, sin)
        if cfg.sink == "learned":
            sink = lay["sink"][i]
        elif cfg.sink == "const":
            sink = torch.full((H,), cfg.sink_init, dtype=F64)
        else:
            sink = None
        a = attention(q, k, v, sink, cfg.attn, cfg.attn_n, cfg.attn_c)
        x = x + a.transpose(1, 2).reshape(B, T, d) @ lay["w_o"][i]
        h2 = _rms_norm(x, lay["ln2"][i] if rms else None, cfg.eps)
        gate, up = h2 @ lay["w_g"][i], h2 @ lay["w_u"][i]
        act = up * torch.sigmoid(up) if cfg.ffn == "swiglu" else _alu(up, cfg.alu_beta)
        x = x + (gate * act) @ lay["w_d"][i]
    hid = _rms_norm(x, params["final_gain"] if rms else None, cfg.eps)
    z = hid.reshape(B * T, d) @ params["embed"].t()
    tgt = targets.reshape(-1)
    if cfg.head == "ce":
        nll = torch.logsumexp(z, -1) - z.gather(1, tgt[:, None])[:, 0]
        return nll.mean(), nll.detach(), nll.mean()
    X = _lean_clamp(z.shape[-1], cfg.head_n)
    logp = torch.log_softmax(cfg.head_n * torch.asinh(torch.clamp(z / cfg.head_c, max=X)), -1)
    lpt = logp.gather(1, tgt[:, None])[:, 0]
    pt = torch.exp(lpt)
    return (1.0 - pt).mean(), pt.detach(), -lpt.mean()
