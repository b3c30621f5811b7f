"""ctypes binding of libalgx.so (the C ABI declared in include/algx.h).

The library is built in-tree by ``algebraic-extra_amd/build.py`` (or
``__graft_entry__.build()``). There is no fallback: every operator of this
package calls into the HIP library and raises if it is missing.
"""

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libalgx.so")

BF16, F32 = 0, 1
SOFTMAX, ASINH = 0, 1
HEAD_CE, HEAD_ALG_CE = 0, 1
ATTN_WS_RAW, ATTN_WS_CLEARED = 0, 1
GLU_ALU, GLU_SILU = 0, 1
PROBE = {"none": 0, "attn_fwd": 1, "attn_bwd": 2, "head_fwd": 3, "head_dz": 4, "head_dh": 5,
         "head_de": 6, "qknorm_fwd": 7, "qknorm_bwd": 8, "rms_norm_fwd": 9, "rms_norm_bwd": 10,
         "alu_fwd": 11, "alu_bwd": 12}

_i32, _i64, _f32, _p = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p


class AttnVariant(ctypes.Structure):
    """algx_attn_variant (include/algx.h)."""
    _fields_ = [("kind", _i32), ("n", _i32), ("shift", _i32), ("fast_rho", _i32),
                ("inv_stat", _i32), ("bounded_scores", _i32), ("precise_output", _i32),
                ("clamp", _f32), ("poly_rho", _i32)]


_VP = ctypes.POINTER(AttnVariant)


class GemmBatch(ctypes.Structure):
    """algx_gemm_batch (include/algx.h)."""
    _fields_ = [("A", _p), ("B", _p), ("D", _p), ("C", _p), ("batch", _i32), ("M", _i32),
                ("N", _i32), ("K", _i32), ("lda", _i64), ("ldb", _i64), ("ldd", _i64),
                ("ldc", _i64), ("stride_a", _i64), ("stride_b", _i64), ("stride_d", _i64),
                ("stride_c", _i64)]

# name -> (restype, argtypes); must match include/algx.h.
SIGNATURES = {
    "algx_last_error": (ctypes.c_char_p, []),
    "algx_version": (_i32, []),
    "algx_selftest_mfma32": (_i32, [_p, _p, _p, _p]),
    "algx_set_probe": (_i32, [_i32, _p, _p]),
    "algx_qknorm_fwd": (_i32, [_p, _p, _p, _i64, _i32, _i32, _f32, _p]),
    "algx_qknorm_bwd_workspace_bytes": (_i64, [_i64, _i32, _i32]),
    "algx_qknorm_bwd": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i32, _i32, _f32, _p]),
    "algx_qknorm_pair_fwd": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i32, _i32, _f32, _p]),
    "algx_qknorm_pair_bwd_workspace_bytes": (_i64, [_i64, _i32, _i32]),
    "algx_qknorm_pair_bwd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i32, _i32,
                                    _f32, _p]),
    "algx_attn_guard_words": (_i32, []),
    "algx_attn_prepare": (_i32, [_p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _f32,
                                 _f32, _f32, _p]),
    "algx_attn_fwd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32,
                             _VP, _VP, _p, _p]),
    "algx_attn_forward_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32]),
    "algx_attn_forward": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i32, _i32, _i32,
                                 _i32, _i32, _f32, _f32, _f32, _VP, _VP, _p]),
    "algx_attn_forward_noalloc": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i32, _i32,
                                         _i32, _i32, _i32, _f32, _f32, _f32, _VP, _VP, _p]),
    "algx_attn_bwd_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32]),
    "algx_attn_bwd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i32, _i32,
                             _i32, _i32, _i32, _i32, _f32, _VP, _VP, _p, _p]),
    "algx_head_fwd_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32]),
    "algx_head_fwd": (_i32, [_p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _f32, _f32,
                             _i32, _p]),
    "algx_head_bwd_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32]),
    "algx_head_bwd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32,
                             _f32, _f32, _i32, _p]),
    "algx_rms_norm_fwd": (_i32, [_p, _p, _p, _i64, _i32, _i32, _f32, _p]),
    "algx_rms_norm_bwd_workspace_bytes": (_i64, [_i64, _i32, _i32]),
    "algx_rms_norm_bwd": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i32, _i32, _f32, _p]),
    "algx_add_rms_norm_fwd": (_i32, [_p, _p, _p, _p, _p, _i64, _i32, _i32, _f32, _p]),
    "algx_add_rms_norm_bwd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _i64, _i32, _i32, _f32, _p]),
    "algx_alu_fwd": (_i32, [_p, _p, _i64, _i32, _f32, _p]),
    "algx_alu_bwd": (_i32, [_p, _p, _p, _i64, _i32, _f32, _p]),
    "algx_alu_glu_fwd": (_i32, [_p, _p, _p, _i64, _i32, _f32, _p]),
    "algx_alu_glu_bwd": (_i32, [_p, _p, _p, _p, _p, _i64, _i32, _f32, _p]),
    "algx_glu_packed_fwd": (_i32, [_p, _p, _i64, _i32, _i32, _i32, _f32, _p]),
    "algx_glu_packed_bwd": (_i32, [_p, _p, _p, _i64, _i32, _i32, _i32, _f32, _p]),
    "algx_swap_axes": (_i32, [_p, _p, _i64, _i64, _i64, _i64, _p]),
    "algx_transpose": (_i32, [_p, _p, _i64, _i64, _i64, _i32, _p]),
    "algx_concat_cast": (_i32, [_p, _p, _i32, _p, _i64, _i32, _p]),
    "algx_split_cast": (_i32, [_p, _p, _p, _i32, _i64, _i32, _p]),
    "algx_muon_momentum": (_i32, [_p, _p, _p, _i64, _f32, _p]),
    "algx_muon_apply": (_i32, [_p, _p, _i64, _i32, _f32, _f32, _p]),
    "algx_adamw_step": (_i32, [_p, _p, _p, _p, _i64, _f32, _f32, _f32, _f32, _f32, _f32, _f32, _p]),
    "algx_ns_normalize_workspace_bytes": (_i64, [_i64, _i64]),
    "algx_ns_normalize": (_i32, [_p, _p, _i64, _i64, _i32, _f32, _p, _p]),
    "algx_gemm_bf16_batched": (_i32, [_p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                      _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                      _f32, _f32, _p]),
    "algx_gemm_bf16_splitk_workspace_bytes": (_i64, [_i32, _i32, _i32]),
    "algx_gemm_bf16_splitk": (_i32, [_p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i64, _i64,
                                     _i64, _i32, _p]),
    "algx_gemm_bf16_grouped": (_i32, [ctypes.POINTER(GemmBatch), _i32, _i32, _i32, _i32, _f32,
                                      _f32, _p]),
    "algx_qk_prologue_fwd": (_i32, [_p, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _i32, _i32,
                                    _i32, _i32, _i32, _f32, _p]),
    "algx_qk_prologue_bwd_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32, _i32]),
    "algx_qk_prologue_bwd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p,
                                    _p, _p, _i32, _i32, _i32, _i32, _i32, _f32, _p]),
}

_lib = None


def load():
    """Load libalgx.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with "
                               "`python algebraic-extra_amd/build.py`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def call(name, *args):
    """Call a status-returning entry point; raise RuntimeError on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.algx_last_error().decode()
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def query(name, *args):
    return getattr(load(), name)(*args)


def ptr(t):
    """Device pointer of a tensor (or None)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def c_ptr(address):
    """A raw device address (an offset into a tensor) as a pointer argument."""
    return ctypes.c_void_p(address)


def stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def dtype_code(dtype):
    import torch
    if dtype == torch.bfloat16:
        return BF16
    if dtype == torch.float32:
        return F32
    raise ValueError(f"unsupported dtype {dtype}")
