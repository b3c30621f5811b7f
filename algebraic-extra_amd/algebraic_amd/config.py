"""Model presets: the softmax baseline and the algebraic model, at four sizes.

Interface of src/algebraic/config.py:8-49 (``SIZES``, ``standard``,
``algebraic``, ``PRESETS``, ``build``). A preset is a size row plus the
architecture switches of its arm; keyword overrides replace any field, which
is how run configurations select kernel implementations (flash attention,
fused head) and sequence length.
"""

from dataclasses import replace
from typing import Dict

from .model import LMConfig

# Width, depth, heads and feed-forward width of each size. The "1b" row has
# d_model 1536: rms_norm handles rows of up to 2048 values.
SIZES: Dict[str, Dict[str, int]] = {
    "proxy": dict(d_model=384, n_layers=8, n_heads=6, d_ff=1024),
    "125m": dict(d_model=768, n_layers=12, n_heads=12, d_ff=2048),
    "350m": dict(d_model=1024, n_layers=24, n_heads=16, d_ff=2688),
    "1b": dict(d_model=1536, n_layers=32, n_heads=24, d_ff=4224),
}

# Architecture switches of each arm.
_STANDARD_ARM = dict(norm="rms", ffn="swiglu", pos="rope", attn="softmax", sink="none",
                     head="ce")
_ALGEBRAIC_ARM = dict(norm="rms", ffn="alu_glu", alu_beta=0.5, pos="cayley_geo", qk_norm=True,
                      attn="asinh", attn_n=16, attn_c=8.0, sink="learned", sink_init=0.0,
                      head="alg_ce", head_n=8, head_c=2.0)


def _preset(arm: Dict, size: str, overrides: Dict) -> LMConfig:
    return replace(LMConfig(**SIZES[size], **arm), **overrides)


def standard(size: str = "proxy", **overrides) -> LMConfig:
    """The comparison arm: gained RMS norms, a SwiGLU feed-forward, rotary
    positions, softmax attention without a sink and a cross-entropy head."""
    return _preset(_STANDARD_ARM, size, overrides)


def algebraic(size: str = "proxy", **overrides) -> LMConfig:
    """The algebraic arm, built from arithmetic and reciprocal roots only:
    gained RMS norms; the gated ALU feed-forward at beta 0.5; Cayley rotations
    at geometric frequencies; normalised queries and keys; attention weights
    rho(s/8)^16 with a learned sink per head; and a head whose likelihood is
    rho(z/2)^8, trained on the gradient of its exact log-likelihood."""
    return _preset(_ALGEBRAIC_ARM, size, overrides)


PRESETS = {"standard": standard, "algebraic": algebraic}


def build(preset: str, size: str, **overrides) -> LMConfig:
    """The named preset at the named size, with field overrides."""
    return PRESETS[preset](size, **overrides)
