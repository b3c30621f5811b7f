"""Pre-norm causal Transformer language model over the algx operators.

Counterpart of ``algebraic.model`` (src/algebraic/model.py) for PyTorch-ROCm:
the same ``LMConfig`` fields, parameter tree (stacked over layers), position
tables, block and head, so that the reference's presets
(``algebraic_amd.config``) build the same architectures. The path's operators
run as HIP kernels of libalgx.so: attention (``flash_attention``, both
``attn_impl`` values), QK-norm, the RMS norms, the ALU-GLU feed-forward
product (and SwiGLU's), the attention prologue (QK-norm, rotation and the
layout change in one pass, for 64-wide heads) and, with
``head_impl="fused"``, the LM head + loss. The projections are plain bf16
GEMMs (hipBLASLt through torch; their weight gradients on libalgx's split-K
GEMM), with q/k/v and gate/up each fused into one
GEMM whose joined bf16 weights are cast once per step (libalgx concat_cast),
and the attention output's head-to-token layout change is a libalgx pass; the
rotation tables, the dense head and, for other head widths, the rotate-half
product are torch ops.

``remat=True`` recomputes each block in the backward
(``torch.utils.checkpoint``), as ``jax.checkpoint`` does (model.py:205-206).
"""

from dataclasses import dataclass
import math
from typing import Any, Dict, Optional

import torch
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint

from .algebraic import add_rms_norm, glu_packed, rms_norm
from .kernels.flash import flash_attention
from .kernels.fused_head import fused_head
from .kernels.prologue import attention_prologue
from .kernels.qk_norm import qk_rms_norm
from .layout import concat_cast, heads_to_tokens, project

F32 = torch.float32
_DTYPES = {"bfloat16": torch.bfloat16, "float32": torch.float32}


@dataclass(frozen=True)
class LMConfig:
    """Field-for-field as model.py:24-67."""
    vocab_size: int = 32768
    d_model: int = 384
    n_layers: int = 8
    n_heads: int = 6
    d_ff: int = 1024
    seq_len: int = 1024
    norm: str = "rms"
    eps: float = 1e-5
    ffn: str = "swiglu"
    alu_beta: float = 1.0
    pos: str = "rope"
    rope_base: float = 10000.0
    rope_fraction: float = 1.0
    attn: str = "softmax"
    attn_n: int = 8
    attn_c: float = 1.0
    sink: str = "none"
    sink_init: float = 0.0
    qk_norm: bool = False
    head: str = "ce"
    head_n: int = 16
    head_c: float = 16.0
    init_std: float = 0.02
    out_init_scale: float = 1.0
    dtype: str = "bfloat16"
    remat: bool = True
    attn_impl: str = "dense"
    flash_block: int = 512
    head_impl: str = "dense"
    head_block_n: int = 128
    head_block_v: int = 512

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads

    @property
    def compute_dtype(self) -> torch.dtype:
        return _DTYPES[self.dtype]

    @property
    def algebraic_path(self) -> bool:
        """True when no transcendental op is used in training (model.py:74-77)."""
        return (self.ffn == "alu_glu" and self.pos.startswith("cayley")
                and self.attn == "asinh" and self.head == "alg_ce")


def count_params(params) -> int:
    return int(sum(t.numel() for t in _leaves(params)))


def _leaves(tree):
    if isinstance(tree, dict):
        for v in tree.values():
            yield from _leaves(v)
    else:
        yield tree


def init_params(cfg: LMConfig, seed: int = 0, device="cuda") -> Dict[str, Any]:
    """Parameter tree of model.py:84-118: float32 leaves, weights ~ N(0, init_std),
    w_o and w_d scaled by out_init_scale, gains one, sink logits sink_init.
    Drawn from torch's generator (the reference draws from jax.random), and
    every leaf requires grad."""
    if cfg.d_model % cfg.n_heads:
        raise ValueError("d_model must be divisible by n_heads")
    gen = torch.Generator(device=device).manual_seed(seed)
    L, d, f, V, H, D = (cfg.n_layers, cfg.d_model, cfg.d_ff, cfg.vocab_size,
                        cfg.n_heads, cfg.head_dim)

    def normal(shape, scale=1.0):
        return torch.randn(shape, generator=gen, device=device, dtype=F32) * (cfg.init_std * scale)

    def ones(shape):
        return torch.ones(shape, device=device, dtype=F32)

    layers = {
        "w_q": normal((L, d, d)),
        "w_k": normal((L, d, d)),
        "w_v": normal((L, d, d)),
        "w_o": normal((L, d, d), cfg.out_init_scale),
        "w_g": normal((L, d, f)),
        "w_u": normal((L, d, f)),
        "w_d": normal((L, f, d), cfg.out_init_scale),
    }
    params: Dict[str, Any] = {"embed": normal((V, d))}
    if cfg.norm == "rms":
        params["embed_gain"] = ones((d,))
        params["final_gain"] = ones((d,))
        layers["ln1"] = ones((L, d))
        layers["ln2"] = ones((L, d))
    elif cfg.norm != "avn":
        raise ValueError(f"unknown norm {cfg.norm!r}")
    if cfg.qk_norm:
        layers["q_gain"] = ones((L, D))
        layers["k_gain"] = ones((L, D))
    if cfg.sink == "learned":
        layers["sink"] = torch.full((L, H), cfg.sink_init, device=device, dtype=F32)
    params["layers"] = layers
    for t in _leaves(params):
        t.requires_grad_(True)
    return params


def decay_mask(params) -> Dict[str, Any]:
    """Weight matrices and the embedding decay; gains and sink logits do not (model.py:121-127)."""
    def rule(name, v):
        if isinstance(v, dict):
            return {k: rule(k, x) for k, x in v.items()}
        return name.startswith("w_") or name == "embed"
    return {k: rule(k, v) for k, v in params.items()}


# ---------------------------------------------------------------------------
# position tables (T, head_dim // 2), float32
# ---------------------------------------------------------------------------

def rope_table(head_dim: int, seq_len: int, base: float = 10000.0, device="cuda"):
    """Trigonometric RoPE tables (standard.py:16-21)."""
    half = head_dim // 2
    theta = 1.0 / (base ** (torch.arange(half, dtype=F32, device=device) / half))
    angles = torch.arange(seq_len, dtype=F32, device=device)[:, None] * theta[None, :]
    return torch.cos(angles), torch.sin(angles)


def cayley_powers(w: torch.Tensor, seq_len: int):
    """Rows ((1 + i w)^2 / (1 + w^2))^m for m < seq_len by binary powering of
    renormalised squarings (algebraic.py:124-149)."""
    w = w.to(F32)
    w2 = w * w
    c = (1.0 - w2) / (1.0 + w2)
    s = (2.0 * w) / (1.0 + w2)
    pos = torch.arange(seq_len, dtype=torch.int32, device=w.device)
    out_c = torch.ones((seq_len, w.shape[0]), dtype=F32, device=w.device)
    out_s = torch.zeros((seq_len, w.shape[0]), dtype=F32, device=w.device)
    bit = 0
    while (1 << bit) < seq_len:
        take = ((pos >> bit) & 1).bool()[:, None]
        new_c = out_c * c - out_s * s
        new_s = out_c * s + out_s * c
        out_c = torch.where(take, new_c, out_c)
        out_s = torch.where(take, new_s, out_s)
        c, s = c * c - s * s, 2.0 * c * s
        inv = torch.rsqrt(c * c + s * s)
        c, s = c * inv, s * inv
        bit += 1
    inv = torch.rsqrt(out_c * out_c + out_s * out_s)
    return out_c * inv, out_s * inv


def cayley_table_geometric(head_dim: int, seq_len: int, base: float = 10000.0,
                           w0: float = 0.5, fraction: float = 1.0, device="cuda"):
    """Geometric grid w_k = w0 base^(-k/half), the ratio by square roots
    (algebraic.py:152-169)."""
    half = head_dim // 2
    levels = int(round(math.log2(half)))
    if 1 << levels != half:
        raise ValueError("geometric Cayley grid needs head_dim/2 to be a power of two")
    root = float(base)
    for _ in range(levels):
        root = math.sqrt(root)
    ratio = 1.0 / root
    active = int(round(fraction * half))
    w = [w0 * ratio ** i if i < active else 0.0 for i in range(half)]
    return cayley_powers(torch.tensor(w, dtype=F32, device=device), seq_len)


def position_tables(cfg: LMConfig, seq_len: Optional[int] = None, device="cuda"):
    """(cos, sin) for cfg.pos (model.py:130-138)."""
    T = seq_len or cfg.seq_len
    if cfg.pos == "rope":
        return rope_table(cfg.head_dim, T, cfg.rope_base, device)
    if cfg.pos == "cayley_geo":
        return cayley_table_geometric(cfg.head_dim, T, cfg.rope_base,
                                      fraction=cfg.rope_fraction, device=device)
    if cfg.pos == "none":
        half = cfg.head_dim // 2
        return (torch.ones((T, half), dtype=F32, device=device),
                torch.zeros((T, half), dtype=F32, device=device))
    raise ValueError(f"unknown position kind {cfg.pos!r}")


def apply_rotary(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half rotation of (B, H, T, D) by (T, D/2) tables (algebraic.py:172-179)."""
    half = x.shape[-1] // 2
    t = x.shape[-2]
    c = cos[:t].to(x.dtype)[None, None]
    s = sin[:t].to(x.dtype)[None, None]
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], dim=-1)


# ---------------------------------------------------------------------------
# blocks
# ---------------------------------------------------------------------------

def _norm(x, gain, cfg: LMConfig):
    """model.py:141-142: learned gain for norm="rms", parameter-free AVN otherwise."""
    return rms_norm(x, gain if cfg.norm == "rms" else None, cfg.eps)


def _qk_norm(x, gain, cfg: LMConfig):
    """rms_norm over the head dimension (model.py:158-159); D = 64 rows take
    the QK-norm kernel, other widths the general row kernel."""
    rows = x.numel() // x.shape[-1]
    if x.shape[-1] == 64 and rows % 8 == 0:
        return qk_rms_norm(x, gain, cfg.eps, block=8)
    return rms_norm(x, gain, cfg.eps)


def _attention(q, k, v, sink_logit, cfg: LMConfig):
    """model.py:144-155. Both attn_impl values run the HIP flash kernels: the
    reference's dense path computes the same function (algebraic.py:207-217,
    standard.py:24-38)."""
    if cfg.attn_impl not in ("dense", "flash"):
        raise ValueError(f"unknown attn_impl {cfg.attn_impl!r}")
    if cfg.attn not in ("softmax", "asinh"):
        raise ValueError(f"unknown attention {cfg.attn!r}")
    return flash_attention(q, k, v, sink_logit, kind=cfg.attn, n=cfg.attn_n, c=cfg.attn_c,
                           block=cfg.flash_block, range_guard=cfg.attn == "asinh")


def _qkv(cfg: LMConfig, cos, sin, h, lp):
    """q, k, v in (B, H, T, D) ready for attention (model.py:166-174).

    With D = 64 one GEMM against [w_q | w_k | w_v] feeds the fused prologue
    kernel (QK-norm, rotation and the layout change in one pass over the
    projections); other head widths take the operators one by one."""
    B, T, d = h.shape
    H, D = cfg.n_heads, cfg.head_dim
    dt = h.dtype
    if D == 64:
        qkv = project(h, lp["w_qkv"])
        gains = (lp["q_gain"], lp["k_gain"]) if cfg.qk_norm else (None, None)
        tabs = (None, None) if cfg.pos == "none" else (cos, sin)
        return attention_prologue(qkv, H, gains[0], gains[1], tabs[0], tabs[1], cfg.eps)
    q = project(h, lp["w_q"].to(dt)).view(B, T, H, D).transpose(1, 2)
    k = project(h, lp["w_k"].to(dt)).view(B, T, H, D).transpose(1, 2)
    v = project(h, lp["w_v"].to(dt)).view(B, T, H, D).transpose(1, 2)
    if cfg.qk_norm:
        q = _qk_norm(q, lp["q_gain"], cfg)
        k = _qk_norm(k, lp["k_gain"], cfg)
    return apply_rotary(q, cos, sin), apply_rotary(k, cos, sin), v


def _add_norm(x, r, gain, cfg: LMConfig):
    """(x + r, norm(x + r)) in one pass; r None: (x, norm(x))."""
    g = gain if cfg.norm == "rms" else None
    if r is None:
        return x, rms_norm(x, g, cfg.eps)
    return add_rms_norm(x, r, g, cfg.eps)


def _block(cfg: LMConfig, cos, sin, x, r, lp):
    """One pre-norm block (model.py:162-191) on the residual stream x + r.

    The block's two residual adds are fused into the norms that read their
    sums: x + r (the previous block's feed-forward output, added here) with
    ln1, and x + attention with ln2. It returns (x, y): the stream after
    attention and this block's feed-forward output, still to be added by the
    next norm. Sums and roundings are those of model.py:177 and :191."""
    H = cfg.n_heads
    x, h = _add_norm(x, r, lp.get("ln1"), cfg)
    q, k, v = _qkv(cfg, cos, sin, h, lp)
    if cfg.sink == "learned":
        sink = lp["sink"].to(F32)
    elif cfg.sink == "const":
        sink = torch.full((H,), cfg.sink_init, dtype=F32, device=x.device)
    else:
        sink = None
    a = heads_to_tokens(_attention(q, k, v, sink, cfg))
    x, h2 = _add_norm(x, project(a, lp["w_o_c"]), lp.get("ln2"), cfg)
    if cfg.ffn not in ("swiglu", "alu_glu"):
        raise ValueError(f"unknown ffn {cfg.ffn!r}")
    # gate and up from one GEMM against [w_g | w_u]; the gated product reads
    # its rows in place and returns the gradient packed the same way.
    gu = project(h2, lp["w_gu"])
    y = glu_packed(gu, "alu" if cfg.ffn == "alu_glu" else "silu", cfg.alu_beta)
    return x, project(y, lp["w_d_c"])


def _joined(parts, dt):
    """torch.cat(parts, -1).to(dt) of float32 stacked weights: one libalgx pass
    each way on the device when every width is a multiple of 4."""
    if (parts[0].is_cuda and all(p.dtype == F32 for p in parts)
            and all(p.shape[-1] % 4 == 0 for p in parts)):
        return concat_cast(parts, dt)
    return torch.cat(parts, dim=-1).to(dt)


def forward_hidden(params, tokens: torch.Tensor, cfg: LMConfig, tables) -> torch.Tensor:
    """Final normalised hidden states (B, T, d) in the compute dtype (model.py:194-208)."""
    cos, sin = tables
    x = F.embedding(tokens, params["embed"]).to(cfg.compute_dtype)
    x = _norm(x, params.get("embed_gain"), cfg)
    # One unbind per stacked leaf: its backward stacks the per-layer gradients
    # in one pass, where indexing t[i] per layer would materialise (and add)
    # a zero-filled full-size gradient for every layer. The matrices are cast
    # to the compute dtype once per step for all layers (the reference casts
    # per block, model.py:167-191: the same values), q/k/v and gate/up
    # concatenated for their fused GEMMs.
    layers = params["layers"]
    dt = cfg.compute_dtype
    per_layer = {name: t.unbind(0) for name, t in layers.items()}
    per_layer["w_o_c"] = layers["w_o"].to(dt).unbind(0)
    per_layer["w_d_c"] = layers["w_d"].to(dt).unbind(0)
    per_layer["w_gu"] = _joined([layers["w_g"], layers["w_u"]], dt).unbind(0)
    if cfg.head_dim == 64:
        per_layer["w_qkv"] = _joined([layers["w_q"], layers["w_k"], layers["w_v"]], dt).unbind(0)
    r = None
    for i in range(cfg.n_layers):
        lp = {name: ts[i] for name, ts in per_layer.items()}
        if cfg.remat:
            x, r = checkpoint(_block, cfg, cos, sin, x, r, lp, use_reentrant=False)
        else:
            x, r = _block(cfg, cos, sin, x, r, lp)
    return _add_norm(x, r, params.get("final_gain"), cfg)[1]


# ---------------------------------------------------------------------------
# heads
# ---------------------------------------------------------------------------

def likelihood_clamp(vocab: int, n: int) -> float:
    """0.25 (1e38 / V)^(1/n) (algebraic.py:277-283)."""
    out = 1e38 / vocab
    k = n
    while k > 1:
        out = math.sqrt(out)
        k //= 2
    return 0.25 * out


def _int_pow(x, n):
    out, base = None, x
    while n:
        if n & 1:
            out = base if out is None else out * base
        n >>= 1
        if n:
            base = base * base
    return out


def _lean_parts(z, n, c, clamp):
    x = torch.clamp(z / c, max=clamp)
    rad = 1.0 + x * x
    r = torch.rsqrt(rad)
    return _int_pow(x + rad * r, n), r


class _LeanLikelihood(torch.autograd.Function):
    """algebraic_likelihood_lean with its custom VJP (algebraic.py:286-320)
    on materialised float32 logits: objective mean(1 - p_t), telemetry p_t,
    gradient (n/c) r (p - y) / N."""

    @staticmethod
    def forward(ctx, logits, targets, n, c):
        z = logits.to(F32)
        w, _ = _lean_parts(z, n, c, likelihood_clamp(z.shape[-1], n))
        wt = w.gather(1, targets[:, None])[:, 0]
        pt = wt / w.sum(-1)
        ctx.save_for_backward(logits, targets)
        ctx.nc = (n, c)
        ctx.mark_non_differentiable(pt)
        return (1.0 - pt).mean(), pt

    @staticmethod
    def backward(ctx, g_obj, g_pt):
        logits, targets = ctx.saved_tensors
        n, c = ctx.nc
        z = logits.to(F32)
        w, r = _lean_parts(z, n, c, likelihood_clamp(z.shape[-1], n))
        p = w / w.sum(-1, keepdim=True)
        y = F.one_hot(targets.long(), z.shape[-1]).to(p.dtype)
        grad = (g_obj * (n / c) / z.shape[0]) * r * (p - y)
        return grad.to(logits.dtype), None, None, None


def head_loss(params, hidden: torch.Tensor, targets: torch.Tensor, cfg: LMConfig):
    """(objective, telemetry) for one micro-batch (model.py:211-231): per-token
    NLL for "ce", target probability for "alg_ce" (no gradient)."""
    N = hidden.shape[0] * hidden.shape[1]
    h = hidden.reshape(N, -1)
    tgt = targets.reshape(N)
    if cfg.head not in ("ce", "alg_ce"):
        raise ValueError(f"unknown head {cfg.head!r}")
    if cfg.head_impl == "fused":
        return fused_head(h, params["embed"], tgt, kind=cfg.head, n=cfg.head_n, c=cfg.head_c,
                          block_n=cfg.head_block_n, block_v=cfg.head_block_v)
    # dense: float32 logits h E^T (preferred_element_type=F32)
    logits = h.to(F32) @ params["embed"].to(h.dtype).to(F32).t()
    if cfg.head == "ce":
        lse = torch.logsumexp(logits, dim=-1)
        nll = lse - logits.gather(1, tgt[:, None].long())[:, 0]
        return nll.mean(), nll.detach()
    return _LeanLikelihood.apply(logits, tgt.long(), cfg.head_n, cfg.head_c)


def telemetry_is_probability(cfg: LMConfig) -> bool:
    return cfg.head != "ce"


def train_objective(params, tokens, targets, cfg: LMConfig, tables):
    """head_loss(forward_hidden(...)): the value the trainer differentiates."""
    return head_loss(params, forward_hidden(params, tokens, cfg, tables), targets, cfg)


__all__ = ["LMConfig", "count_params", "init_params", "decay_mask", "rope_table",
           "cayley_powers", "cayley_table_geometric", "position_tables", "apply_rotary",
           "forward_hidden", "head_loss", "likelihood_clamp", "telemetry_is_probability",
           "train_objective"]
