"""Parity tolerances (stated once, used by every parity test).

* float32: ``|a - b| <= atol + rtol |b|`` with ``rtol = 1e-4`` and
  ``atol = 1e-4 * max|b|``.
* bfloat16 outputs and gradients: max-abs error ``<= 2e-2`` and per-tensor
  relative L2 error ``<= 1e-2``. Where the tensor's largest magnitude is so
  large that one bf16 unit in the last place already exceeds 2e-2 (max|b|
  >= 4, ulp 2^-5), the max-abs bound is that one ulp of max|b|: no bf16 result
  can be closer than half an ulp, and kernel and oracle rounding on either
  side of a value differ by one. Every comparison is recorded and reported at
  the end of the run against the fixed 2e-2.
"""

import numpy as np

F32_RTOL = 1e-4
BF16_MAX_ABS = 2e-2
BF16_REL_L2 = 1e-2

# Every bf16 comparison of the session: (what, max-abs error, max|b|, rel-L2),
# so the max-abs against the fixed 2e-2 can be reported at the end.
BF16_RECORDS = []


def bf16_ulp(x):
    """Spacing of bfloat16 numbers at magnitude x (8 significant bits)."""
    x = float(abs(x))
    if x == 0.0 or not np.isfinite(x):
        return 0.0
    return float(2.0 ** (np.floor(np.log2(x)) - 7))


def to_np(t):
    import torch
    if isinstance(t, torch.Tensor):
        return t.detach().to("cpu", torch.float64).numpy()
    return np.asarray(t, np.float64)


def rel_l2(a, b):
    a, b = to_np(a), to_np(b)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def assert_f32(got, want, rtol=F32_RTOL, what=""):
    a, b = to_np(got), to_np(want)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    assert np.isfinite(a).all(), f"{what}: non-finite values"
    atol = rtol * max(float(np.abs(b).max()), 1e-30)
    err = np.abs(a - b) - (atol + rtol * np.abs(b))
    worst = float(err.max()) if err.size else -1.0
    assert worst <= 0, f"{what}: f32 tolerance exceeded by {worst:.3e} (max|b|={np.abs(b).max():.3e})"


def assert_bf16(got, want, max_abs=BF16_MAX_ABS, rel=BF16_REL_L2, what=""):
    a, b = to_np(got), to_np(want)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    assert np.isfinite(a).all(), f"{what}: non-finite values"
    mae = float(np.abs(a - b).max()) if a.size else 0.0
    mb = float(np.abs(b).max()) if b.size else 0.0
    bound = max(max_abs, bf16_ulp(mb))
    r = rel_l2(a, b)
    BF16_RECORDS.append((what, mae, mb, r))
    assert mae <= bound and r <= rel, f"{what}: max-abs {mae:.3e} (<= {bound:.3e}), rel-L2 {r:.3e} (<= {rel})"


def assert_dtype_close(got, want, dtype, what=""):
    if dtype == "f32":
        assert_f32(got, want, what=what)
    else:
        assert_bf16(got, want, what=what)
