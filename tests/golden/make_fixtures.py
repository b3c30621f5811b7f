"""Write the committed golden fixtures (run from the repository root):

    python tests/golden/make_fixtures.py

cfg0_attention_forward.npz -- BASELINE configs[0], the reference's CPU
plumbing case: asinh-power causal attention forward with QK-norm (RMS over
D, unit gain), B=1, H=4, S=256, D=64, float32, q/k/v ~ N(0, 1) from seed 0.
The reference draws its inputs with jax.random, absent here; these come from
numpy's default_rng(0) and are stored with the outputs. Settings: the model's
algebraic preset (n = 16, c = 8, range guard on, eps = 1e-5). The expected
output is the CPU oracle's (oracle/qknorm.py then oracle/attention.py, float32
roundings); tests/test_golden.py pins it independently against the textbook
dense softmax over n*asinh(s/c).
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import attention as OA  # noqa: E402
from oracle import qknorm as OQ  # noqa: E402

CFG0 = dict(B=1, H=4, T=256, D=64, n=16, c=8.0, eps=1e-5)


def cfg0_inputs():
    rng = np.random.default_rng(0)
    shape = (CFG0["B"], CFG0["H"], CFG0["T"], CFG0["D"])
    return [rng.standard_normal(shape).astype(np.float32) for _ in range(3)]


def cfg0_expected(q, k, v):
    gain = np.ones(CFG0["D"])
    qn = OQ.forward(q, gain, CFG0["eps"], "f32")
    kn = OQ.forward(k, gain, CFG0["eps"], "f32")
    res = OA.flash_attention(qn, kn, np.asarray(v, np.float64), kind="asinh", n=CFG0["n"],
                             c=CFG0["c"], range_guard=True, dtype="f32")
    return res.o.astype(np.float32)


def main():
    q, k, v = cfg0_inputs()
    o = cfg0_expected(q, k, v)
    path = os.path.join(HERE, "cfg0_attention_forward.npz")
    np.savez(path, q=q, k=k, v=v, o=o)
    print(path, o.shape, float(np.abs(o).max()))


if __name__ == "__main__":
    main()
