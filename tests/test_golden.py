"""The committed golden fixture (tests/golden/, made by make_fixtures.py):
BASELINE configs[0], asinh attention forward with QK-norm, B=1, H=4, S=256,
D=64, float32.

CPU: the stored inputs are the seeded draw, the oracle reproduces the stored
output, and that output equals the textbook formula -- softmax over the
compressed logits n*asinh(s/c) of RMS-normalised q, k -- computed here in
float64. GPU: the HIP path (qk_rms_norm, then flash_attention) on the stored
inputs matches the stored output to float32 tolerance.
"""

import math
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_fixtures as MF  # noqa: E402
from _tol import assert_f32  # noqa: E402

FIX = os.path.join(HERE, "golden", "cfg0_attention_forward.npz")


def _load():
    with np.load(FIX, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_fixture_inputs_and_oracle_regression():
    f = _load()
    for name, x in zip(("q", "k", "v"), MF.cfg0_inputs()):
        np.testing.assert_array_equal(f[name], x)
    np.testing.assert_array_equal(MF.cfg0_expected(f["q"], f["k"], f["v"]), f["o"])


def test_fixture_matches_textbook_formula():
    f = _load()
    c, n, eps = MF.CFG0["c"], MF.CFG0["n"], MF.CFG0["eps"]
    q, k, v = (f[x].astype(np.float64) for x in ("q", "k", "v"))
    qn = q / np.sqrt((q * q).mean(-1, keepdims=True) + eps)
    kn = k / np.sqrt((k * k).mean(-1, keepdims=True) + eps)
    T, D = q.shape[-2], q.shape[-1]
    logits = n * np.arcsinh(qn @ np.swapaxes(kn, -1, -2) / (math.sqrt(D) * c))
    logits = np.where(np.tril(np.ones((T, T), bool)), logits, -np.inf)
    p = np.exp(logits - logits.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    want = p @ v
    np.testing.assert_allclose(f["o"], want, rtol=2e-4, atol=2e-5)


@pytest.mark.gpu
def test_hip_path_matches_fixture():
    import torch
    from algebraic_amd.kernels import flash_attention, qk_rms_norm
    f = _load()
    dev = "cuda"
    q, k, v = (torch.from_numpy(f[x]).to(dev) for x in ("q", "k", "v"))
    gain = torch.ones(64, device=dev)
    eps = MF.CFG0["eps"]
    qn = qk_rms_norm(q, gain, eps, block=256)
    kn = qk_rms_norm(k, gain, eps, block=256)
    o = flash_attention(qn, kn, v, kind="asinh", n=MF.CFG0["n"], c=MF.CFG0["c"],
                        range_guard=True)
    torch.cuda.synchronize()
    assert_f32(o, f["o"], what="cfg0 o")
