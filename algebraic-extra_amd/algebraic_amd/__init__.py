"""MI355X (gfx950) kernels for the algebraic-extra hot path.

``algebraic_amd.kernels`` mirrors ``algebraic.kernels`` of the reference
(flash attention, fused LM head + loss, QK RMS norm) on PyTorch-ROCm tensors,
and ``algebraic_amd.algebraic`` the elementwise ops of ``algebraic.algebraic``
the model applies around them (rms_norm, alu, and the fused alu_glu); the
device work runs in libalgx.so (C ABI: include/algx.h).
"""

from . import _lib  # noqa: F401
