"""C-ABI boundary and host-side checks that need no GPU.

* libalgx.so loads and exports every entry point include/algx.h declares;
* host-only queries (workspace sizes, guard words) answer;
* the Python operators raise the reference's ValueErrors before any device
  work (flash.py:796-817, fused_head.py:269-272, qk_norm.py:68-75).
"""

import ctypes
import os
import re

import pytest
import torch

from algebraic_amd import _lib
from algebraic_amd.algebraic import alu, alu_glu, rms_norm
from algebraic_amd.kernels import flash_attention, fused_head, make_variant, qk_rms_norm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "algx.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(algx_\w+)\s*\(", text, re.M)))


def test_header_declarations_match_binding():
    names = _declared()
    assert "algx_attn_fwd" in names and "algx_head_bwd" in names and "algx_qknorm_fwd" in names
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_library_loads_and_exports_every_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.algx_version() == 3
    assert lib.algx_last_error() == b""


def test_host_queries():
    assert _lib.query("algx_attn_guard_words") >= 8
    assert _lib.query("algx_attn_bwd_workspace_bytes", 8, 12, 2048, 64) >= 8 * 12 * 2048 * 64 * 4
    assert _lib.query("algx_qknorm_bwd_workspace_bytes", 1 << 18, 64, 0) > 0
    assert _lib.query("algx_head_fwd_workspace_bytes", 16384, 768, 50304, 0) > 0
    assert _lib.query("algx_head_bwd_workspace_bytes", 16384, 768, 50304, 0) > 0
    assert _lib.query("algx_rms_norm_bwd_workspace_bytes", 16384, 1024, 0) >= 1024 * 4
    assert _lib.query("algx_rms_norm_bwd_workspace_bytes", 0, 1024, 0) == 0


def test_entry_points_reject_bad_arguments_without_a_gpu():
    """Validation happens before any launch: a bad dtype or size returns an error."""
    lib = _lib.load()
    rc = lib.algx_qknorm_fwd(None, None, None, 16, 32, 0, 1e-5, None)
    assert rc != 0 and b"D must be 64" in lib.algx_last_error()
    v = _lib.AttnVariant(kind=1, n=12)
    rc = lib.algx_attn_fwd(None, None, None, None, None, None, None, 1, 1, 128, 64, 0,
                           v, None, None, None)
    assert rc != 0 and b"power of two" in lib.algx_last_error()
    rc = lib.algx_head_fwd(None, None, None, None, None, None, 4, 12, 100, 0, 16, 1.0, 0.0, 0, None)
    assert rc != 0 and b"multiple of 8" in lib.algx_last_error()
    rc = lib.algx_rms_norm_fwd(None, None, None, 4, 100, 0, 1e-5, None)
    assert rc != 0 and b"multiple of 8" in lib.algx_last_error()
    rc = lib.algx_rms_norm_fwd(None, None, None, 4, 2056, 1, 1e-5, None)
    assert rc != 0 and b"at most 2048" in lib.algx_last_error()
    rc = lib.algx_rms_norm_bwd(None, None, None, None, None, None, 0, 64, 0, 1e-5, None)
    assert rc == 0
    g = ctypes.c_void_p(16)
    rc = lib.algx_rms_norm_bwd(g, g, g, g, None, None, 4, 64, 0, 1e-5, None)
    assert rc != 0 and b"dgain" in lib.algx_last_error()
    rc = lib.algx_alu_fwd(None, None, 16, 2, 1.0, None)
    assert rc != 0 and b"dtype" in lib.algx_last_error()
    rc = lib.algx_alu_glu_fwd(ctypes.c_void_p(16), ctypes.c_void_p(24), ctypes.c_void_p(32), 16, 0,
                              1.0, None)
    assert rc != 0 and b"16-byte aligned" in lib.algx_last_error()
    # Attention tensors: a pointer that is not 16-byte aligned (here o) is
    # rejected before any launch, on every entry point.
    v = _lib.AttnVariant(kind=1, n=16)
    a, bad = ctypes.c_void_p(256), ctypes.c_void_p(264)
    rc = lib.algx_attn_fwd(a, a, a, None, bad, None, a, 1, 1, 128, 64, 0, v, None, None, None)
    assert rc != 0 and b"attn_fwd" in lib.algx_last_error()
    assert b"16-byte aligned" in lib.algx_last_error()
    rc = lib.algx_attn_forward(a, a, a, None, a, bad, None, a, None, None, None, 1, 1, 128, 64,
                               0, 1.0, 1.0, 1.0, v, None, None)
    assert rc != 0 and b"attn_forward: q, k, v" in lib.algx_last_error()
    rc = lib.algx_attn_forward(a, a, a, None, a, a, None, a, None, None, bad, 1, 1, 128, 64,
                               0, 1.0, 1.0, 1.0, v, None, None)
    assert rc != 0 and b"attn_forward: q, k, v" in lib.algx_last_error()
    rc = lib.algx_attn_bwd(a, a, a, None, a, None, a, a, bad, a, a, None, a, _lib.ATTN_WS_RAW,
                           1, 1, 128, 64, 0, 1.0, v, None, None, None)
    assert rc != 0 and b"attn_bwd: q, k, v" in lib.algx_last_error()
    rc = lib.algx_attn_bwd(a, a, a, None, a, None, a, a, a, a, a, None, a, 7, 1, 1, 128, 64, 0,
                           1.0, v, None, None, None)
    assert rc != 0 and b"workspace_state" in lib.algx_last_error()
    rc = lib.algx_attn_prepare(a, a, a, None, bad, None, 1, 1, 128, 64, 0, 1.0, 1.0, 1.0, None)
    assert rc != 0 and b"attn_prepare: q, k, v" in lib.algx_last_error()


def test_attn_variant_rejects_polynomial_with_bounded_scores():
    """The polynomial radical never pairs with the guard's unclamped low
    variant (flash.py:835-836 refuses range_guard with poly_rho): the C ABI
    refuses that variant before any launch."""
    lib = _lib.load()
    v = _lib.AttnVariant(kind=1, n=16, shift=0, fast_rho=1, inv_stat=1, bounded_scores=1,
                         clamp=63.75, poly_rho=1)
    rc = lib.algx_attn_fwd(None, None, None, None, None, None, None, 1, 1, 128, 64, 0,
                           v, None, None, None)
    assert rc != 0 and b"bounded_scores=0" in lib.algx_last_error()


def test_noalloc_forward_rejects_sizes_beyond_its_scratch(monkeypatch):
    """More than 65536 forward workgroups (B H T / 128) is refused by the
    no-allocation forward before any other check or launch, on every path
    (the generic-path switch set or not); no device pointer is passed."""
    lib = _lib.load()
    var = _lib.AttnVariant(kind=1, n=16, shift=0, fast_rho=1, inv_stat=1, bounded_scores=1,
                           clamp=63.75)
    guard = ctypes.c_void_p(512)   # never dereferenced: the size check comes first
    for force in (None, "1"):
        if force is None:
            monkeypatch.delenv("ALGX_FORCE_GENERIC", raising=False)
        else:
            monkeypatch.setenv("ALGX_FORCE_GENERIC", force)
        rc = lib.algx_attn_forward_noalloc(None, None, None, None, None, None, None, None, guard,
                                           None, 64, 32, 4352, 64, _lib.BF16, 0.125, 16.0, 1e8,
                                           var, var, None)
        assert rc != 0 and b"65536" in lib.algx_last_error()
        # at the limit the size check passes and the null inputs are refused
        rc = lib.algx_attn_forward_noalloc(None, None, None, None, None, None, None, None, guard,
                                           None, 64, 32, 4096, 64, _lib.BF16, 0.125, 16.0, 1e8,
                                           var, var, None)
        assert rc != 0 and b"null pointer" in lib.algx_last_error()


def test_splitk_gemm_validation_without_a_gpu():
    """algx_gemm_bf16_splitk checks its sizes, chunking and alignment before
    it launches; an empty product launches nothing."""
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    assert lib.algx_gemm_bf16_splitk_workspace_bytes(1024, 3072, 4) == 4 * 1024 * 3072 * 4
    assert lib.algx_gemm_bf16_splitk(None, None, None, None, 0, 64, 64, 1, 1, 64, 64, 64, 4,
                                     None) == 0
    rc = lib.algx_gemm_bf16_splitk(p, p, p, p, 64, 64, 64, 1, 1, 64, 64, 64, 0, None)
    assert rc != 0 and b"splits" in lib.algx_last_error()
    rc = lib.algx_gemm_bf16_splitk(p, p, p, p, 64, 64, 96, 1, 1, 96, 96, 64, 5, None)
    assert rc != 0 and b"multiple of splits" in lib.algx_last_error()
    rc = lib.algx_gemm_bf16_splitk(p, p, p, p, 64, 64, 64, 1, 1, 64, 64, 64, 16, None)
    assert rc != 0 and b"multiples of 8" in lib.algx_last_error()
    rc = lib.algx_gemm_bf16_splitk(p, ctypes.c_void_p(264), p, p, 64, 64, 64, 1, 1, 64, 64, 64, 2,
                                   None)
    assert rc != 0 and b"16-byte aligned" in lib.algx_last_error()
    rc = lib.algx_gemm_bf16_splitk(p, p, p, p, 64, 64, 64, 1, 1, 32, 64, 64, 2, None)
    assert rc != 0 and b"leading dimension" in lib.algx_last_error()
    rc = lib.algx_gemm_bf16_splitk(p, p, p, None, 64, 64, 64, 1, 1, 64, 64, 64, 2, None)
    assert rc != 0 and b"null pointer" in lib.algx_last_error()


def test_grouped_gemm_validation_without_a_gpu():
    """algx_gemm_bf16_grouped checks the group count and every group's
    arguments before it launches; empty groups launch nothing."""
    lib = _lib.load()
    arr = (_lib.GemmBatch * 5)()
    rc = lib.algx_gemm_bf16_grouped(arr, 5, 1, 1, 0, 1.0, 0.0, None)
    assert rc != 0 and b"between 0 and 4" in lib.algx_last_error()
    assert lib.algx_gemm_bf16_grouped(arr, 0, 1, 1, 0, 1.0, 0.0, None) == 0
    assert lib.algx_gemm_bf16_grouped(arr, 2, 1, 1, 0, 1.0, 0.0, None) == 0  # batch 0
    arr[1] = _lib.GemmBatch(16, 16, None, 16, 2, 12, 16, 32, 32, 32, 16, 16, 384, 512, 0, 192)
    rc = lib.algx_gemm_bf16_grouped(arr, 2, 1, 1, 0, 1.0, 0.0, None)
    assert rc != 0 and b"multiples of 8" in lib.algx_last_error()
    arr[1] = _lib.GemmBatch(16, 16, None, 16, 2, 16, 24, 32, 32, 32, 24, 24, 512, 768, 0, 384)
    rc = lib.algx_gemm_bf16_grouped(arr, 2, 1, 1, 1, 1.0, 0.0, None)
    assert rc != 0 and b"M == N" in lib.algx_last_error()


def _t(shape, dtype=torch.bfloat16):
    return torch.zeros(shape, dtype=dtype)


def test_flash_validation_mirrors_reference():
    x = _t((1, 1, 512, 64))
    with pytest.raises(ValueError, match="divisible by blocks"):
        flash_attention(_t((1, 1, 384, 64)), _t((1, 1, 384, 64)), _t((1, 1, 384, 64)),
                        kind="asinh", block=256)
    with pytest.raises(ValueError, match="whole-head residency"):
        flash_attention(x, x, x, kind="asinh", c=8., head_resident=True)   # test_flash_kernel_tpu.py:331-335
    with pytest.raises(ValueError, match="resident backward needs"):
        flash_attention(_t((1, 1, 256, 64)), _t((1, 1, 256, 64)), _t((1, 1, 256, 64)),
                        kind="asinh", resident_bwd=True)
    with pytest.raises(ValueError, match="diagonal backward requires"):
        flash_attention(x, x, x, kind="asinh", resident_bwd=False, diagonal_bwd=True)
    with pytest.raises(ValueError, match="power of two"):
        flash_attention(x, x, x, kind="asinh", n=12)
    with pytest.raises(ValueError, match="unknown attention kernel"):
        flash_attention(x, x, x, kind="relu")
    # poly_rho (flash.py:757-758, :835-836)
    with pytest.raises(ValueError, match="shift=False and n=16"):
        flash_attention(x, x, x, kind="asinh", n=8, shift=False, poly_rho=True)
    with pytest.raises(ValueError, match="range_guard is for exact radical"):
        flash_attention(x, x, x, kind="asinh", n=16, shift=False, poly_rho=True, range_guard=True)


def test_make_variant_matches_reference_defaults():
    v = make_variant("asinh", 16, 8.0, 2048)
    assert abs(v.clamp - 63.75) < 5e-3 and not v.shift and v.inv_stat and v.fast_rho
    assert make_variant("asinh", 32, 8.0, 2048).shift
    assert make_variant("softmax").kind == "softmax"


def test_head_and_norm_validation_mirror_reference():
    h, e, t = _t((256, 64)), torch.zeros((512, 64)), torch.zeros(256, dtype=torch.int64)
    with pytest.raises(ValueError):
        fused_head(h, e, t, kind="mse")
    with pytest.raises(ValueError, match="power of two"):
        fused_head(h, e, t, kind="alg_ce", n=12)
    with pytest.raises(ValueError, match="divisible by block"):
        fused_head(_t((200, 64)), e, t[:200], block_n=128)
    g = torch.ones(64)
    with pytest.raises(ValueError, match="D=64"):
        qk_rms_norm(_t((4, 32)), torch.ones(32))
    with pytest.raises(ValueError, match="float32/BF16"):
        qk_rms_norm(_t((1024, 64), torch.float16), g)
    with pytest.raises(ValueError, match="divisible by a block"):
        qk_rms_norm(_t((1000, 64)), g, block=1024)
    with pytest.raises(ValueError, match="positive"):
        qk_rms_norm(_t((1024, 64)), g, eps=0.0)


def test_elementwise_validation():
    with pytest.raises(NotImplementedError, match="multiple of 8"):
        rms_norm(_t((4, 100)), None)
    with pytest.raises(NotImplementedError, match="at most 2048"):
        rms_norm(_t((4, 2056)), None)
    with pytest.raises(ValueError, match="gain must have shape"):
        rms_norm(_t((4, 64)), torch.ones(32))
    with pytest.raises(ValueError, match="positive"):
        rms_norm(_t((4, 64)), None, eps=0.0)
    with pytest.raises(ValueError, match="float32 or bfloat16"):
        rms_norm(_t((4, 64), torch.float16), None)
    with pytest.raises(ValueError, match="one dtype"):
        alu_glu(_t((4, 64)), _t((4, 64), torch.float32))
    with pytest.raises(ValueError, match="one shape"):
        alu_glu(_t((4, 64)), _t((4, 32)))
    with pytest.raises(ValueError, match="one dtype"):
        alu(_t((4, 64), torch.float64))


def test_layout_validation_without_a_gpu():
    """algx_swap_axes / algx_transpose reject bad arguments before any launch;
    empty moves succeed without touching the device."""
    lib = _lib.load()
    g, h = ctypes.c_void_p(16), ctypes.c_void_p(1 << 20)
    assert lib.algx_swap_axes(g, h, 2, 3, 4, 24, None) != 0
    assert b"multiple of 16" in lib.algx_last_error()
    assert lib.algx_swap_axes(ctypes.c_void_p(24), h, 2, 3, 4, 32, None) != 0
    assert b"16-byte aligned" in lib.algx_last_error()
    assert lib.algx_swap_axes(g, ctypes.c_void_p(48), 2, 3, 4, 32, None) != 0
    assert b"overlap" in lib.algx_last_error()
    assert lib.algx_swap_axes(None, None, 0, 3, 4, 32, None) == 0
    assert lib.algx_transpose(g, h, 2, 3, 4, 8, None) != 0
    assert b"elem_bytes" in lib.algx_last_error()
    assert lib.algx_transpose(g, h, 70000, 3, 4, 2, None) != 0
    assert b"65535" in lib.algx_last_error()
    assert lib.algx_transpose(g, ctypes.c_void_p(20), 1, 3, 4, 2, None) != 0
    assert b"overlap" in lib.algx_last_error()
    assert lib.algx_transpose(None, None, 3, 0, 4, 2, None) == 0
    from algebraic_amd.layout import heads_to_tokens, transpose_last2
    with pytest.raises(ValueError, match="multiple of 16 bytes"):
        heads_to_tokens(_t((1, 2, 3, 4)))
    with pytest.raises(ValueError, match="2 or 4 bytes"):
        transpose_last2(_t((3, 4), torch.float64))


def test_concat_cast_validation_without_a_gpu():
    from algebraic_amd.layout import concat_cast
    with pytest.raises(ValueError, match="1 to 4 parts"):
        concat_cast([_t((2, 4), torch.float32)] * 5, torch.bfloat16)
    with pytest.raises(ValueError, match="float32 parts"):
        concat_cast([_t((2, 4))], torch.bfloat16)
    with pytest.raises(ValueError, match="multiples of 4"):
        concat_cast([_t((2, 6), torch.float32)], torch.bfloat16)
    lib = _lib.load()
    cols = (ctypes.c_int64 * 1)(6)
    parts = (ctypes.c_void_p * 1)(16)
    assert lib.algx_concat_cast(ctypes.cast(parts, ctypes.c_void_p), ctypes.cast(cols, ctypes.c_void_p),
                                1, ctypes.c_void_p(64), 2, 0, None) != 0
    assert b"multiples of 4" in lib.algx_last_error()
