"""Layout moves on the GPU (libalgx algx_swap_axes / algx_transpose).

Both are byte moves, so the check is bit-exact equality with torch's own
permutation of the same tensor: heads_to_tokens against
``a.transpose(1, 2).reshape(B, T, H * D)`` (the reference's
``a.transpose(0, 2, 1, 3).reshape(B, T, d)``, model.py:182) and
transpose_last2 against ``x.transpose(-2, -1)`` (optimizers.py:41, :49), with
ragged shapes that leave partial tiles on both of its paths (register blocks
when both extents are multiples of 16 bytes, LDS tiles otherwise), and their
gradients.
"""

import pytest
import torch

from algebraic_amd.layout import heads_to_tokens, transpose_last2

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _rand(shape, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(shape, device=DEV, generator=g).to(dtype)


@pytest.mark.parametrize("shape,dtype", [
    ((8, 16, 2048, 64), torch.bfloat16),
    ((2, 3, 5, 32), torch.bfloat16),
    ((1, 4, 7, 8), torch.bfloat16),
    ((3, 5, 9, 64), torch.float32),
    ((2, 2, 3, 4), torch.float32),
    ((1, 1, 1, 64), torch.bfloat16),
])
def test_heads_to_tokens_matches_permute(shape, dtype):
    B, H, T, D = shape
    a = _rand(shape, dtype, 11).requires_grad_(True)
    out = heads_to_tokens(a)
    ref = a.detach().transpose(1, 2).reshape(B, T, H * D)
    assert out.shape == (B, T, H * D) and out.is_contiguous()
    assert torch.equal(out, ref)
    g = _rand((B, T, H * D), dtype, 12)
    (da,) = torch.autograd.grad(out, a, g)
    assert torch.equal(da, g.view(B, T, H, D).transpose(1, 2))


def test_heads_to_tokens_noncontiguous_input():
    a = _rand((2, 6, 4, 64), torch.bfloat16, 13)[:, ::2]
    assert not a.is_contiguous()
    assert torch.equal(heads_to_tokens(a), a.transpose(1, 2).reshape(2, 4, 3 * 64))


@pytest.mark.parametrize("shape,dtype", [
    ((72, 1024, 2688), torch.bfloat16),
    ((96, 1024, 1024), torch.bfloat16),
    ((3, 65, 130), torch.bfloat16),
    ((5, 63, 17), torch.float32),
    ((2, 2688, 1024), torch.float32),
    ((1, 1, 1), torch.bfloat16),
    ((7, 1), torch.float32),
    ((4, 2, 3, 100, 70), torch.bfloat16),
    ((3, 72, 40), torch.bfloat16),
    ((2, 36, 20), torch.float32),
    ((1, 8, 8), torch.bfloat16),
])
def test_transpose_matches_torch(shape, dtype):
    x = _rand(shape, dtype, 21).requires_grad_(True)
    y = transpose_last2(x)
    assert y.is_contiguous() and torch.equal(y, x.detach().transpose(-2, -1))
    g = _rand(y.shape, dtype, 22)
    (dx,) = torch.autograd.grad(y, x, g)
    assert torch.equal(dx, g.transpose(-2, -1))


def test_transpose_empty():
    x = torch.empty((3, 0, 5), device=DEV, dtype=torch.bfloat16)
    assert transpose_last2(x).shape == (3, 5, 0)


@pytest.mark.parametrize("widths,lead,dtype", [
    ((1024, 1024, 1024), (24, 1024), torch.bfloat16),
    ((2688, 2688), (24, 1024), torch.bfloat16),
    ((8, 12, 4), (3, 5), torch.bfloat16),
    ((16, 20), (2, 7), torch.float32),
    ((4,), (1, 1), torch.bfloat16),
])
def test_concat_cast_matches_torch(widths, lead, dtype):
    """concat_cast == torch.cat(parts, -1).to(dtype) bit for bit (float32 ->
    bf16 rounds to nearest even in both), and its gradient is the split of
    the incoming gradient cast to float32."""
    from algebraic_amd.layout import concat_cast
    parts = [_rand(lead + (w,), torch.float32, 30 + i).requires_grad_(True)
             for i, w in enumerate(widths)]
    out = concat_cast(parts, dtype)
    assert out.dtype == dtype and torch.equal(out, torch.cat([p.detach() for p in parts], -1).to(dtype))
    g = _rand(out.shape, dtype, 40)
    grads = torch.autograd.grad(out, parts, g)
    for got, want in zip(grads, g.float().split(list(widths), dim=-1)):
        assert got.dtype == torch.float32 and torch.equal(got, want)
