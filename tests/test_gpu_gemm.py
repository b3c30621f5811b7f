"""algx_gemm_bf16_batched (the Newton-Schulz products, optimizers.py:46-60)
against a float32 torch reference of the same bf16 inputs."""

import pytest
import torch

from algebraic_amd import optimizers as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ref(A, B, a_kc, b_kc, D, alpha, beta):
    a = A.float() if a_kc else A.float().transpose(1, 2)
    b = B.float() if b_kc else B.float().transpose(1, 2)
    c = alpha * torch.bmm(a, b.transpose(1, 2).contiguous())
    return c + beta * D.float() if D is not None else c


def _check(got, want):
    err = (got.float() - want).abs().max().item()
    scale = want.abs().max().item()
    # bf16 output rounding (2^-8 relative) on float32 sums of bf16 products
    assert err <= 8e-3 * scale + 1e-3, (err, scale)


@pytest.mark.parametrize("a_kc,b_kc", [(True, True), (True, False), (False, True), (False, False)])
@pytest.mark.parametrize("batch,M,N,K", [(3, 264, 520, 96), (8, 256, 256, 1024), (2, 40, 8, 72),
                                         (5, 520, 264, 200), (2, 264, 520, 32), (2, 256, 256, 64)])
def test_batched_gemm_layouts(a_kc, b_kc, batch, M, N, K):
    """Ragged tiles (M, N not multiples of 256), K a multiple of 32 (direct-to-
    LDS stages) or only of 8 (register-staged stages), batches that do and do
    not take the XCD-grouped workgroup order, every operand layout."""
    g = torch.Generator(device=DEV).manual_seed(M + N + K)
    A = torch.randn((batch, M, K) if a_kc else (batch, K, M), generator=g, device=DEV).bfloat16()
    B = torch.randn((batch, N, K) if b_kc else (batch, K, N), generator=g, device=DEV).bfloat16()
    D = torch.randn((batch, M, N), generator=g, device=DEV).bfloat16()
    got = O.gemm_bf16_batched(A, B, a_kc=a_kc, b_kc=b_kc, D=D, alpha=-0.5, beta=1.5)
    _check(got, _ref(A, B, a_kc, b_kc, D, -0.5, 1.5))
    got = O.gemm_bf16_batched(A, B, a_kc=a_kc, b_kc=b_kc)
    _check(got, _ref(A, B, a_kc, b_kc, None, 1.0, 0.0))


def test_batched_gemm_in_place_combination():
    """D may be the output itself (each element is read before it is written)."""
    g = torch.Generator(device=DEV).manual_seed(7)
    A = torch.randn((4, 128, 256), generator=g, device=DEV).bfloat16()
    C = torch.randn((4, 128, 128), generator=g, device=DEV).bfloat16()
    want = _ref(A, A, True, True, C, 2.0315, -4.775)
    O.gemm_bf16_batched(A, A, a_kc=True, b_kc=True, D=C, alpha=2.0315, beta=-4.775, out=C)
    _check(C, want)


def test_batched_gemm_rejects_bad_shapes():
    A = torch.zeros((2, 12, 16), device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="multiples of 8"):
        O.gemm_bf16_batched(A, A, a_kc=True, b_kc=True)
    with pytest.raises(ValueError, match="do not chain"):
        O.gemm_bf16_batched(A, torch.zeros((2, 8, 24), device=DEV, dtype=torch.bfloat16),
                            a_kc=True, b_kc=True)


def test_newton_schulz_products_match_torch_iteration():
    """The native iteration against the same iteration on torch bmm/baddbmm
    (float32 sums of the same bf16 products), at the model's wide shape."""
    g = torch.Generator(device=DEV).manual_seed(3)
    G = torch.randn((8, 1024, 2688), generator=g, device=DEV)
    X = torch.empty(G.shape, dtype=torch.bfloat16, device=DEV)
    O._normalize_into(G, X, 1e-7)
    got = O._ns_iterate(X.clone(), 5)
    a, b, c = O._NS_ABC
    Y = X.clone()
    for _ in range(5):
        A = torch.bmm(Y, Y.transpose(1, 2).contiguous())
        Bm = torch.baddbmm(A, A, A, beta=b, alpha=c)
        Y = torch.baddbmm(Y, Bm, Y, beta=a, alpha=1.0)
    for _ in range(2):
        Y = torch.baddbmm(Y, torch.bmm(Y, Y.transpose(1, 2).contiguous()), Y, beta=1.5, alpha=-0.5)
    rel = ((got.float() - Y.float()).norm() / Y.float().norm()).item()
    assert rel <= 2e-2, rel


@pytest.mark.parametrize("batch,M,K", [(3, 520, 96), (8, 1024, 256), (2, 264, 72)])
def test_batched_gemm_symmetric_products(batch, M, K):
    """symmetric=True forms only the tiles on and above the diagonal and
    mirrors them: X X^T (ragged tile counts; K = 72 takes the full schedule)
    and c A A + b A with A symmetric."""
    g = torch.Generator(device=DEV).manual_seed(M + K)
    X = torch.randn((batch, M, K), generator=g, device=DEV).bfloat16()
    A = O.gemm_bf16_batched(X, X, a_kc=True, b_kc=True, symmetric=True)
    _check(A, _ref(X, X, True, True, None, 1.0, 0.0))
    if K % 32 == 0:
        # off-diagonal 256 x 256 blocks are exact mirrors
        for i in range(0, M, 256):
            for j in range(i + 256, M, 256):
                assert torch.equal(A[:, j:j + 256, i:i + 256], A[:, i:i + 256, j:j + 256].transpose(1, 2))
    As = ((A.float() + A.float().transpose(1, 2)) * 0.5).bfloat16()
    Bm = O.gemm_bf16_batched(As, As, a_kc=True, b_kc=False, D=As, alpha=2.0315, beta=-4.775,
                             symmetric=True)
    _check(Bm, _ref(As, As, True, False, As, 2.0315, -4.775))


def test_batched_gemm_symmetric_needs_square():
    A = torch.zeros((2, 16, 32), device=DEV, dtype=torch.bfloat16)
    B = torch.zeros((2, 24, 32), device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="M == N"):
        O.gemm_bf16_batched(A, B, a_kc=True, b_kc=True, symmetric=True)



@pytest.mark.parametrize("a_kc,b_kc,sym", [(True, True, True), (True, False, True),
                                          (True, False, False), (False, True, False),
                                          (False, False, False)])
def test_grouped_launch_equals_one_call_per_batch(a_kc, b_kc, sym):
    """algx_gemm_bf16_grouped: batches of different shapes (ragged tiles,
    batch counts that do and do not take the XCD-grouped order, K of both
    stage kinds when not symmetric) in one launch give exactly what one
    algx_gemm_bf16_batched call per batch gives."""
    g = torch.Generator(device=DEV).manual_seed(11 + 2 * a_kc + b_kc + 4 * sym)
    shapes = ([(8, 264, 264, 96), (3, 520, 520, 200), (16, 256, 256, 64)] if sym else
              [(8, 264, 520, 96), (3, 40, 8, 72), (5, 520, 264, 200), (16, 256, 256, 1024)])
    problems = []
    for batch, M, N, K in shapes:
        A = torch.randn((batch, M, K) if a_kc else (batch, K, M), generator=g, device=DEV).bfloat16()
        if sym:
            B = A
        else:
            B = torch.randn((batch, N, K) if b_kc else (batch, K, N), generator=g, device=DEV).bfloat16()
        D = torch.randn((batch, M, N), generator=g, device=DEV)
        if sym:
            D = (D + D.transpose(1, 2)) * 0.5
        problems.append((A, B, D.bfloat16().contiguous()))
    if sym and not b_kc:
        # c A A + b A with A symmetric (the Newton-Schulz form)
        problems = [(D, D, D) for _, _, D in problems]
    outs = O.gemm_bf16_grouped([(A, B, D, None) for A, B, D in problems], a_kc=a_kc, b_kc=b_kc,
                               alpha=-0.75, beta=1.25, symmetric=sym)
    for (A, B, D), got in zip(problems, outs):
        want = O.gemm_bf16_batched(A, B, a_kc=a_kc, b_kc=b_kc, D=D, alpha=-0.75, beta=1.25,
                                   symmetric=sym)
        assert torch.equal(got, want)
    # without D, and a single group
    outs = O.gemm_bf16_grouped([(A, B, None, None) for A, B, _ in problems[:1]], a_kc=a_kc,
                               b_kc=b_kc, symmetric=sym)
    A, B, _ = problems[0]
    assert torch.equal(outs[0], O.gemm_bf16_batched(A, B, a_kc=a_kc, b_kc=b_kc, symmetric=sym))


def test_grouped_launch_rejects():
    A = torch.zeros((2, 16, 32), device=DEV, dtype=torch.bfloat16)
    B = torch.zeros((2, 24, 32), device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="M == N"):
        O.gemm_bf16_grouped([(A, A, None, None), (A, B, None, None)], a_kc=True, b_kc=True,
                            symmetric=True)
    with pytest.raises(ValueError, match="at most 4"):
        O.gemm_bf16_grouped([(A, A, None, None)] * 5, a_kc=True, b_kc=True)
    with pytest.raises(ValueError, match="beta needs"):
        O.gemm_bf16_grouped([(A, A, None, None)], a_kc=True, b_kc=True, beta=1.0)
    assert O.gemm_bf16_grouped([], a_kc=True, b_kc=True) == []


def test_newton_schulz_groups_in_lockstep_equal_separate_runs():
    """newton_schulz_many iterates its shape groups together (one grouped
    launch per product): the result equals each batch iterated alone."""
    g = torch.Generator(device=DEV).manual_seed(5)
    Xs = []
    for shape in ((16, 1024, 1024), (8, 1024, 2688), (3, 264, 520)):
        G = torch.randn(shape, generator=g, device=DEV)
        X = torch.empty(shape, dtype=torch.bfloat16, device=DEV)
        O._normalize_into(G, X, 1e-7)
        Xs.append(X)
    together = O._ns_iterate_many([X.clone() for X in Xs], 5)
    for X, got in zip(Xs, together):
        assert torch.equal(got, O._ns_iterate(X.clone(), 5))


def _splitk(A, B, a_kc, b_kc, splits):
    from algebraic_amd import _lib
    M = A.shape[0] if a_kc else A.shape[1]
    K = A.shape[1] if a_kc else A.shape[0]
    N = B.shape[0] if b_kc else B.shape[1]
    C = torch.full((M, N), float("nan"), device=DEV, dtype=torch.bfloat16)
    ws = torch.full((_lib.query("algx_gemm_bf16_splitk_workspace_bytes", M, N, splits) // 4,),
                    float("nan"), device=DEV)
    _lib.call("algx_gemm_bf16_splitk", _lib.ptr(A), _lib.ptr(B), _lib.ptr(C), _lib.ptr(ws), M, N,
              K, int(a_kc), int(b_kc), A.shape[1], B.shape[1], N, splits, _lib.stream())
    return C


@pytest.mark.parametrize("a_kc,b_kc", [(True, True), (True, False), (False, True), (False, False)])
@pytest.mark.parametrize("M,N,K,splits", [(264, 520, 1024, 4), (1024, 1024, 4096, 16),
                                          (40, 8, 96, 4), (520, 264, 2048, 1), (256, 768, 640, 5)])
def test_splitk_gemm_matches_float32(a_kc, b_kc, M, N, K, splits):
    """algx_gemm_bf16_splitk: bf16(opA opB^T) from float32 sums over K cut into
    chunks (direct-to-LDS stages when a chunk is whole 32-row stages,
    register-staged otherwise; ragged tiles; every operand layout), into
    outputs and a workspace that start as NaN; two calls agree bit for bit."""
    g = torch.Generator(device=DEV).manual_seed(M * 3 + N + K + splits)
    A = torch.randn((M, K) if a_kc else (K, M), generator=g, device=DEV).bfloat16()
    B = torch.randn((N, K) if b_kc else (K, N), generator=g, device=DEV).bfloat16()
    C = _splitk(A, B, a_kc, b_kc, splits)
    a = A.float() if a_kc else A.float().t()
    b = B.float() if b_kc else B.float().t()
    want = a @ b.t()
    assert torch.isfinite(C.float()).all()
    err = (C.float() - want).abs()
    # one bf16 rounding of float32 sums of exact bf16 products
    assert (err <= 2 ** -8 * want.abs() + 5e-5 * (a.abs() @ b.abs().t())).all(), err.max().item()
    assert torch.equal(C, _splitk(A, B, a_kc, b_kc, splits))


def test_splitk_gemm_rejects_bad_arguments():
    from algebraic_amd import _lib
    A = torch.zeros((64, 64), device=DEV, dtype=torch.bfloat16)
    ws = torch.zeros(64 * 64 * 16, device=DEV)
    for splits, msg in ((0, "splits"), (3, "multiple of splits"), (16, "multiples of 8")):
        with pytest.raises(RuntimeError, match=msg):
            _lib.call("algx_gemm_bf16_splitk", _lib.ptr(A), _lib.ptr(A), _lib.ptr(A), _lib.ptr(ws),
                      64, 64, 64, 1, 1, 64, 64, 64, splits, _lib.stream())


def test_project_gradients_match_torch():
    """layout.project (the model's projections): forward and input gradient
    are torch's product; the weight gradient (split-K, float32 sums rounded
    once to bf16) matches torch's bf16 autodiff within one bf16 rounding."""
    from algebraic_amd.layout import project
    g = torch.Generator(device=DEV).manual_seed(11)
    for (B, T, din, dout) in ((2, 1024, 1024, 3072), (1, 4096, 2688, 1024), (3, 160, 256, 264)):
        x = torch.randn((B, T, din), generator=g, device=DEV).bfloat16().requires_grad_(True)
        w = (0.02 * torch.randn((din, dout), generator=g, device=DEV)).bfloat16().requires_grad_(True)
        dy = torch.randn((B, T, dout), generator=g, device=DEV).bfloat16()
        out = project(x, w)
        dx, dw = torch.autograd.grad(out, (x, w), dy)
        xr, wr = x.detach().clone().requires_grad_(True), w.detach().clone().requires_grad_(True)
        ref = xr @ wr
        rdx, rdw = torch.autograd.grad(ref, (xr, wr), dy)
        assert torch.equal(out, ref)
        assert (dx.float() - rdx.float()).abs().max().item() <= 2 ** -7 * rdx.float().abs().max().item()
        want = x.detach().float().reshape(-1, din).t() @ dy.float().reshape(-1, dout)
        err = (dw.float() - want).abs().max().item()
        assert err <= 2 ** -7 * want.abs().max().item(), err
        assert (rdw.float() - want).abs().max().item() <= 2 ** -7 * want.abs().max().item()

def _spread_rows(rows, ld):
    """rows (R, K) laid out ld elements apart in one flat bf16 buffer."""
    R, K = rows.shape
    flat = torch.zeros((R - 1) * ld + K, dtype=torch.bfloat16, device=DEV)
    for r in range(R):
        flat[r * ld: r * ld + K] = rows[r]
    return flat


def test_operands_beyond_32bit_lane_offsets_take_the_staged_path():
    """An A operand whose 8 rows lie 4e8 elements apart spans 5.6 GB, past the
    32-bit lane offsets of the direct-to-LDS loads: the batched and split-K
    products take the register-staged stages for it (K = 64 would otherwise
    take the direct-to-LDS ring) and match the float32 reference. A wrong
    path choice would wrap the offsets inside the allocation and give wrong
    values, not a fault."""
    from algebraic_amd import _lib
    M, N, K, lda = 8, 256, 64, 400_000_000
    g = torch.Generator(device=DEV).manual_seed(21)
    rows = torch.randn((M, K), generator=g, device=DEV).bfloat16()
    B = torch.randn((N, K), generator=g, device=DEV).bfloat16()
    big = _spread_rows(rows, lda)
    want = rows.float() @ B.float().t()
    C = torch.full((M, N), float("nan"), device=DEV, dtype=torch.bfloat16)
    _lib.call("algx_gemm_bf16_batched", _lib.ptr(big), _lib.ptr(B), None, _lib.ptr(C), 1, M, N,
              K, 1, 1, 0, lda, K, 0, N, 0, 0, 0, 0, 1.0, 0.0, _lib.stream())
    _check(C, want)
    C2 = torch.full((M, N), float("nan"), device=DEV, dtype=torch.bfloat16)
    ws = torch.empty((_lib.query("algx_gemm_bf16_splitk_workspace_bytes", M, N, 1) // 4,),
                     device=DEV)
    _lib.call("algx_gemm_bf16_splitk", _lib.ptr(big), _lib.ptr(B), _lib.ptr(C2), _lib.ptr(ws), M,
              N, K, 1, 1, lda, K, N, 1, _lib.stream())
    _check(C2, want)
    del big
    torch.cuda.empty_cache()
