"""Reference-compatible operators: flash_attention, fused_head, qk_rms_norm
(and qk_rms_norm_pair, the q and k norms in one launch)."""

from .flash import Variant, flash_attention, make_variant  # noqa: F401
from .fused_head import fused_head  # noqa: F401
from .qk_norm import qk_rms_norm, qk_rms_norm_pair  # noqa: F401
