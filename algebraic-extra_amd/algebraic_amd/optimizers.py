"""Muon + AdamW, cautious AdamW and the hybrid, on PyTorch-ROCm tensors.

Counterpart of ``algebraic.optimizers`` (src/algebraic/optimizers.py): the
same ``newton_schulz_5``, ``is_muon_param``, ``make_cosine_schedule`` and
``get_optimizer(name, lr, ...) -> (init_fn, step_fn)`` with the reference's
update rules. The parameter trees are the model's dicts of float32 tensors;
``step_fn`` updates parameters and state in place and returns them (the
functional signature of the reference, without copying 1.4 GB per step).

The Newton-Schulz products run as batched GEMMs over the layer-stacked
weights (hipBLASLt through torch). ``ns_dtype`` selects their input type:
bfloat16 (default; the reference's float32 matmuls run as single bfloat16
passes on its TPUs at default precision) or float32. Every transpose the
iteration needs is materialised by libalgx's tiled transpose kernel (one
read and one write of the batch) rather than by a strided torch copy, and
Muon's elementwise steps around it (momentum with the Nesterov look-ahead,
and the decayed update from the orthogonalised matrix) are single libalgx
passes over the float32 state.
"""

import math
from typing import Any, Callable, Dict, Optional, Tuple

import torch

from . import _lib
from .layout import transpose_last2

F32 = torch.float32


def _mT(x: torch.Tensor) -> torch.Tensor:
    """x.transpose(-2, -1), contiguous: libalgx's tiled transpose for device
    tensors (torch's strided copy of the same moves runs 2-3x slower there);
    tensors on the host take torch's copy."""
    return transpose_last2(x) if x.is_cuda else x.transpose(-2, -1).contiguous()


def _aligned(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _muon_momentum(g: torch.Tensor, m: torch.Tensor, mu: float) -> torch.Tensor:
    """m <- mu m + (1 - mu) g in place; returns the look-ahead (1 - mu) g + mu m
    (optimizers.py:200-201). Contiguous float32 device state: one libalgx
    pass."""
    if m.is_cuda and m.dtype == F32 and m.is_contiguous() and m.data_ptr() % 16 == 0:
        g = _aligned(g.to(F32))
        look = torch.empty_like(m)
        _lib.call("algx_muon_momentum", _lib.ptr(g), _lib.ptr(m), _lib.ptr(look), m.numel(),
                  float(mu), _lib.stream())
        return look
    m.mul_(mu).add_(g, alpha=1.0 - mu)
    return g.mul(1.0 - mu).add_(m, alpha=mu)


def _muon_apply(p: torch.Tensor, o: torch.Tensor, decay_fac: float, step: float) -> None:
    """p <- p * decay_fac - step * o in place (optimizers.py:203-204), o in the
    Newton-Schulz dtype. Contiguous float32 device parameters: one libalgx
    pass."""
    if p.is_cuda and p.dtype == F32 and p.is_contiguous() and p.data_ptr() % 16 == 0:
        o = _aligned(o)
        _lib.call("algx_muon_apply", _lib.ptr(p), _lib.ptr(o), p.numel(),
                  _lib.dtype_code(o.dtype), float(decay_fac), float(step), _lib.stream())
        return
    if decay_fac != 1.0:
        p.mul_(decay_fac)
    p.add_(o.to(F32), alpha=-step)


def _fused_ok(*ts) -> bool:
    return all(t.is_cuda and t.dtype == F32 and t.is_contiguous() and t.data_ptr() % 16 == 0
               for t in ts)


def _adamw_step(p, g, m, v, b1, b2, c1, c2, eps, decay_fac, lr) -> None:
    """The Adam leaf update of optimizers.py:222-226 in place, one libalgx pass
    (m, v and p read and written once, g read once)."""
    g = _aligned(g.to(F32))
    _lib.call("algx_adamw_step", _lib.ptr(p), _lib.ptr(g), _lib.ptr(m), _lib.ptr(v), p.numel(),
              float(b1), float(b2), float(c1), float(c2), float(eps), float(decay_fac),
              float(lr), _lib.stream())


_NS_ABC = (3.4445, -4.7750, 2.0315)


def _normalize_into(X: torch.Tensor, out: torch.Tensor, eps: float) -> None:
    """out <- X / sqrt(sum(X^2) + eps) per (m, n) matrix of X (k, m, n), cast to
    out's dtype (optimizers.py:44-45). Device tensors: two libalgx passes
    (per-matrix sums of squares, then the scaled copy) with no float32
    intermediate."""
    X = X.to(F32).contiguous()
    if X.is_cuda and out.is_contiguous() and out.dtype in (torch.bfloat16, F32):
        K, MN = X.shape[0], X.shape[1] * X.shape[2]
        ws = torch.empty(max(1, _lib.query("algx_ns_normalize_workspace_bytes", K, MN)),
                         dtype=torch.uint8, device=X.device)
        _lib.call("algx_ns_normalize", _lib.ptr(X), _lib.ptr(out), K, MN,
                  _lib.dtype_code(out.dtype), float(eps), _lib.ptr(ws), _lib.stream())
        return
    norm = torch.sqrt((X * X).sum(dim=(-2, -1), keepdim=True) + eps)
    out.copy_(X / norm)


def _ns_wide(X: torch.Tensor, steps: int, eps: float, ns_dtype: torch.dtype) -> torch.Tensor:
    """Newton-Schulz on a batch (k, m, n), m <= n, without the aspect factor."""
    Xn = torch.empty(X.shape, dtype=ns_dtype, device=X.device)
    _normalize_into(X, Xn, eps)
    return _ns_iterate(Xn, steps)


def _gemm_problem(A, B, a_kc, b_kc, D, out, who):
    """One batch of the GEMM core's products: checked shapes, the output
    (allocated when not given) and its algx_gemm_batch descriptor."""
    kb, ra, ca = A.shape
    M, K = (ra, ca) if a_kc else (ca, ra)
    N, Kb = (B.shape[1], B.shape[2]) if b_kc else (B.shape[2], B.shape[1])
    if B.shape[0] != kb or Kb != K:
        raise ValueError(f"{who}: shapes {tuple(A.shape)} and {tuple(B.shape)} do not chain")
    for t in (A, B) + tuple(x for x in (D, out) if x is not None):
        if t.dtype != torch.bfloat16 or not t.is_cuda or not t.is_contiguous():
            raise ValueError(f"{who}: operands must be contiguous bf16 device tensors")
    for name, t in (("D", D), ("out", out)):
        if t is not None and tuple(t.shape) != (kb, M, N):
            raise ValueError(f"{who}: {name} must be (batch, M, N)")
    if out is None:
        out = torch.empty((kb, M, N), dtype=torch.bfloat16, device=A.device)
    desc = _lib.GemmBatch(A.data_ptr(), B.data_ptr(), D.data_ptr() if D is not None else None,
                          out.data_ptr(), kb, M, N, K, A.shape[2], B.shape[2], N, N, ra * ca,
                          B.shape[1] * B.shape[2], M * N, M * N)
    return desc, out


def gemm_bf16_batched(A: torch.Tensor, B: torch.Tensor, *, a_kc: bool, b_kc: bool,
                      D: Optional[torch.Tensor] = None, alpha: float = 1.0, beta: float = 0.0,
                      out: Optional[torch.Tensor] = None, symmetric: bool = False) -> torch.Tensor:
    """C[i] = alpha * opA(A[i]) opB(B[i])^T + beta * D[i] on libalgx's MFMA
    GEMM core (algx_gemm_bf16_batched), bf16 in and out, float32 sums.

    A, B: contiguous bf16 (k, r, c) batches. opA is A[i] itself ([M][K]) when
    a_kc, else A[i]^T (A stored [K][M]); opB is B[i] ([N][K]) when b_kc, else
    B[i]^T. So C = A B^T for (True, True) and C = A B for (True, False).
    ``symmetric`` states that C is symmetric (the product and D): only the
    tiles on and above the diagonal are formed, then mirrored."""
    g, out = _gemm_problem(A, B, a_kc, b_kc, D, out, "gemm_bf16_batched")
    _lib.call("algx_gemm_bf16_batched", g.A, g.B, g.D, g.C, g.batch, g.M, g.N, g.K,
              int(a_kc), int(b_kc), int(symmetric), g.lda, g.ldb, g.ldd, g.ldc, g.stride_a,
              g.stride_b, g.stride_d, g.stride_c, float(alpha),
              float(beta if D is not None else 0.0), _lib.stream())
    return out


def gemm_bf16_grouped(problems, *, a_kc: bool, b_kc: bool, alpha: float = 1.0,
                      beta: float = 0.0, symmetric: bool = False):
    """gemm_bf16_batched over up to four batches of different shapes in one
    launch (algx_gemm_bf16_grouped): ``problems`` is a list of (A, B, D, out)
    with D and out optional (None), the layouts, symmetry and coefficients
    shared. Returns the outputs, equal bit for bit to one
    gemm_bf16_batched call per batch."""
    if len(problems) > 4:
        raise ValueError("gemm_bf16_grouped: at most 4 batches per launch")
    descs, outs = [], []
    for A, B, D, out in problems:
        g, out = _gemm_problem(A, B, a_kc, b_kc, D, out, "gemm_bf16_grouped")
        if D is None and beta != 0.0:
            raise ValueError("gemm_bf16_grouped: beta needs every batch's D")
        descs.append(g)
        outs.append(out)
    arr = (_lib.GemmBatch * max(1, len(descs)))(*descs)
    _lib.call("algx_gemm_bf16_grouped", arr, len(descs), int(a_kc), int(b_kc), int(symmetric),
              float(alpha), float(beta), _lib.stream())
    return outs


def _ns_native_ok(X: torch.Tensor) -> bool:
    m, n = X.shape[-2:]
    return (X.is_cuda and X.dtype == torch.bfloat16 and X.is_contiguous() and
            m % 8 == 0 and n % 8 == 0 and X.data_ptr() % 16 == 0)


def _ns_iterate(X: torch.Tensor, steps: int) -> torch.Tensor:
    """The iteration on a normalised, contiguous batch (k, m, n), m <= n. On
    the native path X is also a working buffer (overwritten)."""
    return _ns_iterate_many([X], steps)[0]


def _ns_iterate_many(Xs_in, steps: int):
    """The iteration on normalised, contiguous batches (k, m, n), m <= n, of
    any mix of shapes.

    Each update is one GEMM with its linear combination folded into the
    GEMM's own alpha/beta: B = b A + c A A and X <- a X + B X, and
    X <- 1.5 X - 0.5 (X X^T) X for the refinements. bf16 device batches run
    on libalgx's GEMM core, all batches of one product in one launch
    (gemm_bf16_grouped, four at most): X X^T reads X k-contiguous on both
    sides (no transpose is formed), A A and B X read their second operand as
    [k][n], and every product writes a buffer of its own (no self copy). The
    input batches are working buffers of the native path (the iterate
    ping-pongs between each input and one more buffer of its shape), so their
    contents are overwritten."""
    a, b, c = _NS_ABC
    if 0 < len(Xs_in) <= 4 and all(_ns_native_ok(X) for X in Xs_in):
        st = []
        for X in Xs_in:
            k, m, n = X.shape
            A = torch.empty((k, m, m), dtype=X.dtype, device=X.device)
            st.append({"A": A, "B": torch.empty_like(A), "X": [X, torch.empty_like(X)]})
        if all(t.data_ptr() % 16 == 0 for e in st for t in (e["A"], e["B"], e["X"][1])):
            cur = 0

            def gram():
                # A = X X^T: symmetric, upper-triangle tiles only
                gemm_bf16_grouped([(e["X"][cur], e["X"][cur], None, e["A"]) for e in st],
                                  a_kc=True, b_kc=True, symmetric=True)

            def update(mat, acc_coef, own_coef):
                # X <- own_coef X + acc_coef (mat X), into the other buffer
                nonlocal cur
                gemm_bf16_grouped([(e[mat], e["X"][cur], e["X"][cur], e["X"][1 - cur])
                                   for e in st], a_kc=True, b_kc=False, alpha=acc_coef,
                                  beta=own_coef)
                cur = 1 - cur

            for _ in range(steps):
                gram()
                # B = b A + c A A, symmetric as A is
                gemm_bf16_grouped([(e["A"], e["A"], e["A"], e["B"]) for e in st], a_kc=True,
                                  b_kc=False, alpha=c, beta=b, symmetric=True)
                update("B", 1.0, a)
            for _ in range(2):
                gram()
                update("A", -0.5, 1.5)
            return [e["X"][cur] for e in st]
    if len(Xs_in) > 1:
        return [_ns_iterate_many([X], steps)[0] for X in Xs_in]
    X = Xs_in[0]

    def gram(x):
        return torch.bmm(x, _mT(x))

    for _ in range(steps):
        A = gram(X)
        Bm = torch.baddbmm(A, A, A, beta=b, alpha=c)
        X = torch.baddbmm(X, Bm, X, beta=a, alpha=1.0)
    for _ in range(2):
        X = torch.baddbmm(X, gram(X), X, beta=1.5, alpha=-0.5)
    return [X]


def newton_schulz_5(G: torch.Tensor, steps: int = 5, eps: float = 1e-7,
                    ns_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Orthogonalise the trailing (M, N) matrices of G (optimizers.py:27-64):
    Frobenius pre-normalisation, ``steps`` quintic iterations with
    (a, b, c) = (3.4445, -4.7750, 2.0315), two order-3 Schulz refinements,
    and the aspect-ratio factor sqrt(max(1, M/N)). Returns float32."""
    if G.ndim < 2:
        return G
    M, N = G.shape[-2], G.shape[-1]
    X = G.reshape((-1, M, N))
    if M > N:
        X = _mT(X.to(F32))
    X = _ns_wide(X, steps, eps, ns_dtype)
    if M > N:
        X = _mT(X)
    return (X.to(F32) * math.sqrt(max(1.0, float(M) / float(N)))).reshape(G.shape)


def newton_schulz_many(Gs, steps: int = 5, eps: float = 1e-7,
                       ns_dtype: torch.dtype = torch.bfloat16):
    """newton_schulz_5 of every tensor in Gs, the matrices of equal (oriented)
    shape run as one batch: the model's 7 stacked weights become two batches
    ([w_q | w_k | w_v | w_o] and [w_g | w_u | w_d^T])."""
    return [(y.to(F32) * sc if sc != 1.0 else y.to(F32)).reshape(G.shape)
            for G, (y, sc) in zip(Gs, _newton_schulz_unscaled(Gs, steps, eps, ns_dtype))]


def _newton_schulz_unscaled(Gs, steps, eps, ns_dtype):
    """(X, scale) per tensor of Gs: X the orthogonalised matrix in ns_dtype
    and G's layout, scale the aspect factor sqrt(max(1, M / N)) still to be
    applied (optimizers.py:63-64)."""
    groups: Dict[Tuple[int, int], list] = {}
    for i, G in enumerate(Gs):
        M, N = G.shape[-2], G.shape[-1]
        X = G.reshape((-1, M, N))
        if M > N:
            X = _mT(X.to(F32))
        groups.setdefault(tuple(X.shape[-2:]), []).append((i, X))
    out = [None] * len(Gs)
    batches = []
    for items in groups.values():
        # each matrix normalised straight into its slice of the batch
        k_all = sum(x.shape[0] for _, x in items)
        m, n = items[0][1].shape[-2:]
        batch = torch.empty((k_all, m, n), dtype=ns_dtype, device=items[0][1].device)
        k0 = 0
        for _, x in items:
            _normalize_into(x, batch[k0:k0 + x.shape[0]], eps)
            k0 += x.shape[0]
        batches.append(batch)
    # the shape groups iterate together, four per GEMM launch
    Ys = []
    for i in range(0, len(batches), 4):
        Ys += _ns_iterate_many(batches[i:i + 4], steps)
    for items, Y in zip(groups.values(), Ys):
        k0 = 0
        for i, x in items:
            y = Y[k0:k0 + x.shape[0]]
            k0 += x.shape[0]
            G = Gs[i]
            M, N = G.shape[-2], G.shape[-1]
            if M > N:
                y = _mT(y)
            out[i] = (y.reshape(G.shape), math.sqrt(max(1.0, float(M) / float(N))))
    return out


def is_muon_param(path, param) -> bool:
    """Layer weight matrices take Muon; embedding, gains, sinks and biases the
    Adam family (optimizers.py:67-89). ``path``: the key path (a tuple of
    names) of the leaf."""
    if path:
        key = str(path[-1] if isinstance(path, (list, tuple)) else path)
        if key == "embed":
            return False
        if key.startswith("w_"):
            return True
        if key.startswith("ln") or key.endswith("_gain") or key == "sink" or "bias" in key:
            return False
    return getattr(param, "ndim", 0) >= 2


def make_cosine_schedule(peak_lr: float, total_steps: int, warmup_fraction: float,
                         min_lr_ratio: float) -> Callable[[int], float]:
    """Linear warmup then cosine decay to min_lr_ratio * peak (optimizers.py:92-115)."""
    warm = (float(warmup_fraction) if warmup_fraction >= 1
            else max(1.0, float(round(warmup_fraction * total_steps))))
    floor = peak_lr * min_lr_ratio
    total_t = float(total_steps)

    def schedule(step) -> float:
        t = float(step) + 1.0
        if t < warm:
            return peak_lr * min(1.0, t / warm)
        prog = min(max((t - warm) / max(1.0, total_t - warm), 0.0), 1.0)
        return floor + (peak_lr - floor) * 0.5 * (1.0 + math.cos(math.pi * prog))

    return schedule


def _flatten(tree, prefix=()):
    if isinstance(tree, dict):
        out = []
        for k, v in tree.items():
            out.extend(_flatten(v, prefix + (k,)))
        return out
    return [(prefix, tree)]


def _get(tree, path):
    for k in path:
        tree = tree[k]
    return tree


class OptState:
    """count, first moments m, second moments v (None for Muon leaves), keyed
    by the leaf's key path (optimizers.py:20-24)."""

    def __init__(self, count: int, m: Dict, v: Dict):
        self.count, self.m, self.v = count, m, v


def get_optimizer(name: str, lr: float, weight_decay: float = 0.1, total_steps: int = 1000,
                  warmup_fraction: float = 0.02, min_lr_ratio: float = 0.1, b1: float = 0.9,
                  b2: float = 0.95, adam_eps: float = 1e-8, muon_lr: Optional[float] = None,
                  muon_wd: Optional[float] = None, muon_momentum: float = 0.95,
                  muon_steps: int = 5, cautious_eps: float = 1e-3,
                  ns_dtype: torch.dtype = torch.bfloat16, **kwargs: Any
                  ) -> Tuple[Callable, Callable]:
    """(init_fn, step_fn) for 'muon_adamw', 'cadamw' or 'hybrid_muon_cadamw'
    (optimizers.py:118-246)."""
    opt_name = name.lower().strip()
    valid = ("muon_adamw", "cadamw", "hybrid_muon_cadamw")
    if opt_name not in valid:
        raise ValueError(f"Unknown optimizer: {name}. Choices: {valid}")
    m_lr = lr if muon_lr is None else muon_lr
    m_wd = weight_decay if muon_wd is None else muon_wd
    adam_schedule = make_cosine_schedule(lr, total_steps, warmup_fraction, min_lr_ratio)
    muon_schedule = make_cosine_schedule(m_lr, total_steps, warmup_fraction, min_lr_ratio)
    uses_muon = opt_name in ("muon_adamw", "hybrid_muon_cadamw")

    def init_fn(params) -> OptState:
        m, v = {}, {}
        for path, p in _flatten(params):
            m[path] = torch.zeros_like(p, dtype=F32)
            muon = uses_muon and is_muon_param(path, p)
            v[path] = None if muon else torch.zeros_like(p, dtype=F32)
        return OptState(0, m, v)

    @torch.no_grad()
    def step_fn(step: int, params, grads, opt_state: OptState, decay_mask):
        adam_lr = adam_schedule(step)
        muon_lr_t = muon_schedule(step)
        t = float(step + 1)
        c1, c2 = 1.0 - b1 ** t, 1.0 - b2 ** t
        muon_jobs = []
        for path, p in _flatten(params):
            g = _get(grads, path)
            if g is None:
                continue
            g = g.to(F32)
            m, v = opt_state.m[path], opt_state.v[path]
            decay = bool(_get(decay_mask, path))
            if uses_muon and is_muon_param(path, p):
                # m <- mu m + (1 - mu) g and the Nesterov look-ahead, orthogonalised below
                muon_jobs.append((p, decay, _muon_momentum(g, m, muon_momentum)))
                continue
            decay_fac = 1.0 - adam_lr * weight_decay if decay else 1.0
            if opt_name == "muon_adamw" and _fused_ok(p, m, v):
                _adamw_step(p, g, m, v, b1, b2, c1, c2, adam_eps, decay_fac, adam_lr)
                continue
            m.mul_(b1).add_(g, alpha=1.0 - b1)
            v.mul_(b2).addcmul_(g, g, value=1.0 - b2)
            u = (m / c1) / (torch.sqrt(v / c2) + adam_eps)
            if opt_name in ("cadamw", "hybrid_muon_cadamw"):
                mask = (u * g > 0.0).to(F32)
                u = u * (mask / torch.clamp(mask.mean(), min=cautious_eps))
            if decay:
                p.mul_(1.0 - adam_lr * weight_decay)
            p.add_(u, alpha=-adam_lr)
        if muon_jobs:
            ortho = _newton_schulz_unscaled([look for _, _, look in muon_jobs], muon_steps, 1e-7,
                                            ns_dtype)
            for (p, decay, _), (o, sc) in zip(muon_jobs, ortho):
                _muon_apply(p, o, 1.0 - muon_lr_t * m_wd if decay else 1.0, muon_lr_t * sc)
        opt_state.count += 1
        return params, opt_state

    return init_fn, step_fn


def grads_of(params) -> Dict:
    """The .grad tree of a parameter tree (None where a leaf has no gradient)."""
    if isinstance(params, dict):
        return {k: grads_of(v) for k, v in params.items()}
    return params.grad


__all__ = ["OptState", "newton_schulz_5", "newton_schulz_many", "is_muon_param",
           "make_cosine_schedule", "get_optimizer", "grads_of"]
