"""bench.py's contract pieces that need no GPU: the one-GPU refusal and the
FLOP conventions its TFLOP/s figures divide by (the reference harness's
bench_attention.py:50,65 and bench_head.py:36)."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert res.returncode == 2
    assert "one GPU" in (res.stdout + res.stderr)


def test_attention_flop_convention():
    # causal forward: 2 products of 2·T·T·D flops per head, half of them kept
    B, H, T, D = 8, 12, 2048, 64
    fwd = bench.attn_flops_fwd(B, H, T, D)
    assert fwd == 2 * (2 * B * H * T * T * D) / 2
    # fwd + bwd = 3.5 x forward (the backward's five products and the
    # forward's two, over the forward's two): 180.39 GFLOP at configs[1]
    assert round(3.5 * fwd / 1e9, 2) == 180.39


def test_head_flop_convention():
    # logits, dh and dE: three N x d x V products, 3.798 TFLOP at configs[2]
    N, d, V = 16384, 768, 50304
    assert bench.head_flops(N, d, V) == 3 * (2 * N * d * V)
    assert round(bench.head_flops(N, d, V) / 1e12, 3) == 3.798
