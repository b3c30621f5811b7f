"""MI355X (gfx950) kernels for the algebraic-extra hot path.

``algebraic_amd.kernels`` mirrors ``algebraic.kernels`` of the reference
(flash attention, fused LM head + loss, QK RMS norm) on PyTorch-ROCm tensors;
the device work runs in libalgx.so (C ABI: include/algx.h).
"""

from . import _lib  # noqa: F401
