"""HIP-graph capture of the hot path's steps (torch.cuda.graph over the
autograd functions of libalgx).

The entry points launch only kernels on the caller's stream (no allocation,
no host synchronisation, no memset nodes), so a forward + backward step can
be captured once and replayed. Each test replays the graph several times with
eager GPU work and synchronisations between the replays, and checks every
replay against the eager step on the same inputs: bit for bit where every
element is written once in a fixed order, and within one unit in the last
place where float32 atomics add in a run-dependent order before a bf16 cast
(the attention's dQ), and to float32 rounding for the sink gradient (a
float32 atomic sum).
"""

import pytest
import torch

from algebraic_amd.kernels import flash_attention, fused_head

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _capture(step):
    """Warm up on a side stream, then capture one step; returns (graph, outputs)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    return graph, outs


def _ulp(x, mantissa_bits):
    """One unit in the last place of |x| for a format with that many explicit
    mantissa bits (7 for bf16, 23 for float32)."""
    mag = x.abs().clamp_min(torch.finfo(torch.float32).tiny)
    return torch.exp2(torch.floor(torch.log2(mag)) - mantissa_bits)


def _close(got, want, mode):
    """exact: bit for bit. bf16_ulp: within one bf16 ulp (a float32 sum whose
    order varies, rounded once to bf16). f32_sum: a float32 sum over many
    terms whose order varies, to 1e-5 of its largest element."""
    if mode == "exact":
        return torch.equal(got, want)
    a, b = got.float(), want.float()
    if mode == "bf16_ulp":
        bound = _ulp(torch.maximum(a.abs(), b.abs()), 7)
    else:
        bound = 1e-5 * b.abs().max() + 1e-7
    return bool(((a - b).abs() <= bound).all())


def _replays_match(graph, checks):
    """checks: (name, graph output, eager output, mode) per output."""
    for i in range(4):
        # unrelated eager work between replays
        junk = torch.randn(1 << 20, device=DEV)
        junk.mul_(2.0).sum().item()
        graph.replay()
        torch.cuda.synchronize()
        for name, got, want, mode in checks:
            assert _close(got, want, mode), f"replay {i}: {name} ({mode})"


@pytest.mark.parametrize("with_sink", [False, True])
def test_attention_step_in_a_graph_replays_like_eager(with_sink):
    """T = 1024: the queries of the last 256 get dQ contributions from four
    256-key blocks, added by float32 atomics in a run-dependent order."""
    g = torch.Generator(device=DEV).manual_seed(11)
    B, H, T, D = 2, 4, 1024, 64
    q, k, v, do = (torch.randn((B, H, T, D), device=DEV, generator=g).bfloat16() for _ in range(4))
    q, k, v = (x.requires_grad_(True) for x in (q, k, v))
    sink = (0.5 * torch.randn(H, device=DEV, generator=g)).requires_grad_(True) if with_sink else None
    ins = (q, k, v) + ((sink,) if with_sink else ())

    def step():
        o = flash_attention(q, k, v, sink, kind="asinh", n=16, c=8.0, range_guard=True)
        return (o,) + torch.autograd.grad(o, ins, do)

    eager = [t.detach().clone() for t in step()]
    graph, outs = _capture(step)
    # o, dk and dv are written once per element; dq is the bf16 cast of a
    # float32 atomic sum, dsink a float32 atomic sum
    names = ("o", "dq", "dk", "dv", "dsink")
    modes = {"o": "exact", "dq": "bf16_ulp", "dk": "exact", "dv": "exact", "dsink": "f32_sum"}
    checks = [(nm, got, want, modes[nm]) for nm, got, want in zip(names, outs, eager)]
    assert len(checks) == len(outs)
    _replays_match(graph, checks)


def test_fused_head_step_in_a_graph_replays_like_eager():
    """Every output of the head step is written once per element in a fixed
    order (the statistics are merged in chunk order, dh and dE are plain
    stores of one token chunk), so every replay equals the eager step bit for
    bit."""
    g = torch.Generator(device=DEV).manual_seed(12)
    N, d, V = 1024, 256, 4096
    h = torch.randn((N, d), device=DEV, generator=g).bfloat16().requires_grad_(True)
    E = (0.1 * torch.randn((V, d), device=DEV, generator=g)).bfloat16().requires_grad_(True)
    t = torch.randint(0, V, (N,), device=DEV, generator=g)

    def step():
        obj, tel = fused_head(h, E, t, kind="alg_ce", n=8, c=2.0)
        return (obj, tel) + torch.autograd.grad(obj, (h, E))

    eager = [x.detach().clone() for x in step()]
    graph, outs = _capture(step)
    names = ("obj", "telemetry", "dh", "dE")
    checks = [(nm, got, want, "exact") for nm, got, want in zip(names, outs, eager)]
    assert len(checks) == len(outs)
    _replays_match(graph, checks)
