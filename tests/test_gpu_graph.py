"""HIP-graph capture of the hot path's steps (torch.cuda.graph over the
autograd functions of libalgx).

The entry points launch only kernels on the caller's stream (no allocation,
no host synchronisation, no memset nodes), so a forward + backward step can
be captured once and replayed. Each test replays the graph several times with
eager GPU work and synchronisations between the replays, and checks every
replay against the eager step on the same inputs: bit for bit where the
kernels are deterministic, to float32 rounding for dQ, dsink and dE (their
float32 atomics add in a run-dependent order).
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


def _replays_match(graph, outs, eager, exact):
    for i in range(4):
        # unrelated eager work between replays
        junk = torch.randn(1 << 20, device=DEV)
        junk.mul_(2.0).sum().item()
        graph.replay()
        torch.cuda.synchronize()
        for name, got, want in zip(exact + tuple(f"x{j}" for j in range(len(outs))), outs, eager):
            if name in exact:
                assert torch.equal(got, want), f"replay {i}: {name}"
            else:
                assert torch.allclose(got.float(), want.float(), rtol=1e-5, atol=1e-6), f"replay {i}: {name}"


@pytest.mark.parametrize("with_sink", [False, True])
def test_attention_step_in_a_graph_replays_like_eager(with_sink):
    g = torch.Generator(device=DEV).manual_seed(11)
    B, H, T, D = 2, 4, 512, 64
    q, k, v, do = (torch.randn((B, H, T, D), device=DEV, generator=g).bfloat16() for _ in range(4))
    q, k, v = (x.requires_grad_(True) for x in (q, k, v))
    sink = (0.5 * torch.randn(H, device=DEV, generator=g)).requires_grad_(True) if with_sink else None
    ins = (q, k, v) + ((sink,) if with_sink else ())

    def step():
        o = flash_attention(q, k, v, sink, kind="asinh", n=16, c=8.0, range_guard=True)
        return (o,) + torch.autograd.grad(o, ins, do)

    eager = [t.detach().clone() for t in step()]
    graph, outs = _capture(step)
    # o, dk and dv are written once per element (deterministic); dq and dsink
    # come from float32 atomics
    _replays_match(graph, outs, eager, exact=("o",))
    for i, (got, want) in enumerate(zip(outs, eager)):
        if i in (0, 2, 3):
            assert torch.equal(got, want), i
        else:
            assert torch.allclose(got.float(), want.float(), rtol=1e-5, atol=1e-6), i


def test_fused_head_step_in_a_graph_replays_like_eager():
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
    _replays_match(graph, outs, eager, exact=("obj",))
    for i, (got, want) in enumerate(zip(outs, eager)):
        assert torch.allclose(got.float(), want.float(), rtol=1e-5, atol=1e-6), i
