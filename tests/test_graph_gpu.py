"""GPU tests of the operators under HIP graph capture.

The library allocates, frees and synchronises nothing and records no memset
(its work lists are written by kernels), so a forward + backward captured in
a graph must replay to the eager results. Each test replays its graph
several times, clearing the graph's outputs and running eager work of its
own between replays, and compares every replay with the eager run bitwise
(the kernels are deterministic).
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from flash_spacetime_amd import (
        flash_spacetime_attention, flash_spacetime_attention_varlen, flash_spacetime_backward,
        flash_spacetime_forward,
    )

DEV = "cuda"
REPLAYS = 3


def _padded(batch, length, heads, dim, chans, seed, dtype=torch.bfloat16):
    gen = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=gen)  # noqa: E731
    q, k, v, do = (rn(batch, heads, length, dim).to(DEV, dtype) for _ in range(4))
    feats = torch.cat([(torch.rand(batch, length, 3, generator=gen) - 0.5) * 1000,
                       torch.rand(batch, length, 1, generator=gen) * 2e4], -1).to(DEV)
    w = (rn(dim, chans) / chans ** 0.5).to(DEV)
    b = (rn(dim) * 0.02).to(DEV)
    lens = torch.randint(1, length + 1, (batch,), generator=gen)
    lens[0] = length
    return q, k, v, do, feats, w, b, lens.to(DEV, torch.int32)


def _warm_up(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_launchers_replay_in_a_graph(dtype):
    q, k, v, do, feats, w, b, sl = _padded(4, 200, 12, 32, 16, 31, dtype)

    def run():
        out, lse = flash_spacetime_forward(q, k, v, feats, w, b, sl)
        rowsum = torch.empty_like(lse)
        grads = flash_spacetime_backward(q, k, v, feats, w, b, sl, lse, do, rowsum=rowsum)
        return (out, lse, rowsum, *grads)

    ref = [t.clone() for t in run()]
    _warm_up(run)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = run()
    for i in range(REPLAYS):
        for t in static:
            t.fill_(float("nan"))
        eager = run()  # the program's own work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, got, want, again in zip(("out", "lse", "rowsum", "dq", "dk", "dv", "dW", "db"), static,
                                          ref, eager):
            assert torch.equal(got, want), f"replay {i}: {name}"
            assert torch.equal(again, want), f"eager run {i}: {name}"


def test_autograd_step_replays_in_a_graph():
    """Whole-step capture: the autograd op's forward and backward, with the
    parameter gradients, in one graph (packed events)."""
    gen = torch.Generator().manual_seed(41)
    lens = [300, 1, 77, 160]
    total = sum(lens)
    rn = lambda *s: torch.randn(*s, generator=gen)  # noqa: E731
    q0, k0, v0, do = (rn(total, 8, 32).to(DEV, torch.bfloat16) for _ in range(4))
    feats = torch.cat([(torch.rand(total, 3, generator=gen) - 0.5) * 1000,
                       torch.rand(total, 1, generator=gen) * 2e4], -1).to(DEV)
    cu = torch.tensor([0, 300, 301, 378, 538], dtype=torch.int32, device=DEV)
    leaves = [x.clone().requires_grad_(True) for x in (q0, k0, v0)]
    w = (rn(32, 16) / 4).to(DEV).requires_grad_(True)
    b = (rn(32) * 0.02).to(DEV).requires_grad_(True)
    params = [*leaves, w, b]

    def step():
        for p in params:
            p.grad = None
        out = flash_spacetime_attention_varlen(*leaves, feats, w, b, cu)
        out.backward(do)
        return out

    ref_out = step().detach().clone()
    ref_grads = [p.grad.clone() for p in params]
    _warm_up(step)
    for p in params:
        p.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = flash_spacetime_attention_varlen(*leaves, feats, w, b, cu)
        out.backward(do)
    grads = [p.grad for p in params]
    for i in range(REPLAYS):
        out.detach().fill_(float("nan"))
        for g in grads:
            g.fill_(float("nan"))
        eager = flash_spacetime_attention_varlen(*[x.detach() for x in leaves], feats, w.detach(), b.detach(), cu)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.detach(), ref_out), f"replay {i}: out"
        assert torch.equal(eager, ref_out), f"eager run {i}: out"
        for name, g, want in zip(("dq", "dk", "dv", "dW", "db"), grads, ref_grads):
            assert torch.equal(g, want), f"replay {i}: {name}"


def test_padded_autograd_op_in_a_graph_matches_eager():
    q, k, v, do, feats, w, b, sl = _padded(3, 130, 4, 16, 32, 43)
    leaves = [x.clone().requires_grad_(True) for x in (q, k, v)]

    def fwd_bwd():
        for x in leaves:
            x.grad = None
        out = flash_spacetime_attention(*leaves, feats, w, b, sl)
        out.backward(do)
        return out

    ref_out = fwd_bwd().detach().clone()
    ref_grads = [x.grad.clone() for x in leaves]
    _warm_up(fwd_bwd)
    for x in leaves:
        x.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = flash_spacetime_attention(*leaves, feats, w, b, sl)
        out.backward(do)
    for i in range(REPLAYS):
        for x in leaves:
            x.grad.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.detach(), ref_out), f"replay {i}: out"
        for g, want in zip((x.grad for x in leaves), ref_grads):
            assert torch.equal(g, want), f"replay {i}"
