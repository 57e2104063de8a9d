"""HIP-graph capture and torch.compile of the attention ops.

The entry points enqueue on the caller's stream, allocate through torch's
caching allocator and never synchronise the host, so a fwd+bwd step can be
captured once and replayed (the reference's capture path:
oops/attention/triangle/nested.py:126-134).  Replays are checked against
eager calls on the same inputs, with eager work and synchronisations between
replays.  torch.compile traces the front-end and keeps the custom ops opaque
(the reference's compiled test modes, test_triangle_attention.py:330-419).
"""

import pytest
import torch

from oops_amd import pair_bias_attention, triangle_attention

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _inputs(seed, dtype=torch.bfloat16, n=96, ending=True):
    g = torch.Generator().manual_seed(seed)
    base = [torch.randn(1, n, n, 4, 32, generator=g).to(dtype).to(DEV) for _ in range(3)]
    q, k, v = (b.transpose(1, 2) if ending else b for b in base)
    bias = torch.randn(1, 1, 4, n, n, generator=g).to(dtype).to(DEV)
    mask = (torch.rand(1, n, n, generator=g) > 0.1).to(DEV)
    dout = torch.randn(1, n, n, 4, 32, generator=g).to(dtype).to(DEV)
    return q, k, v, mask, bias, dout


def _eager(q, k, v, mask, bias, dout):
    leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v, bias)]
    # clone() keeps the ending-node strides of q/k/v (dense, non-overlapping)
    out = triangle_attention(leaves[0], leaves[1], leaves[2], mask, leaves[3])
    return (out.detach(), *torch.autograd.grad(out, leaves, dout))


def test_graph_capture_replay():
    q, k, v, mask, bias, dout = _inputs(0)
    static = [t.clone() for t in (q, k, v, bias)]
    for t in static:
        t.requires_grad_(True)
    s_mask, s_dout = mask.clone(), dout.clone()

    def step():
        out = triangle_attention(static[0], static[1], static[2], s_mask, static[3])
        return (out, *torch.autograd.grad(out, static, s_dout))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    for replay in range(3):
        new = _inputs(10 + replay)
        with torch.no_grad():
            for dst, src in zip((*static, s_mask, s_dout), (new[0], new[1], new[2], new[4], new[3], new[5])):
                dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        want = _eager(*new)
        torch.cuda.synchronize()
        for got, ref in zip(captured, want):
            torch.testing.assert_close(got, ref, atol=0, rtol=0)


@pytest.mark.parametrize("ending", [False, True])
def test_compile_matches_eager(ending):
    q, k, v, mask, bias, dout = _inputs(3, ending=ending, n=80)

    def run(q_, k_, v_, m_, b_):
        return triangle_attention(q_, k_, v_, m_, b_)

    compiled = torch.compile(run, fullgraph=True)
    leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v, bias)]
    out = compiled(leaves[0], leaves[1], leaves[2], mask, leaves[3])
    grads = torch.autograd.grad(out, leaves, dout)
    want = _eager(q, k, v, mask, bias, dout)
    for got, ref in zip((out, *grads), want):
        torch.testing.assert_close(got, ref, atol=0, rtol=0)


def test_pair_bias_compile_matches_eager():
    g = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn(6, 4, 70, 32, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3))
    mask = (torch.rand(6, 70, generator=g) > 0.2).to(DEV)
    bias = torch.randn(1, 4, 70, 70, generator=g).to(torch.bfloat16).to(DEV)
    dout = torch.randn(6, 4, 70, 32, generator=g).to(torch.bfloat16).to(DEV)

    def run(q_, k_, v_, m_, b_):
        return pair_bias_attention(q_, k_, v_, m_, b_)

    results = []
    for fn in (run, torch.compile(run, fullgraph=True)):
        leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v, bias)]
        out = fn(leaves[0], leaves[1], leaves[2], mask, leaves[3])
        results.append((out.detach(), *torch.autograd.grad(out, leaves, dout)))
    for got, ref in zip(*results):
        torch.testing.assert_close(got, ref, atol=0, rtol=0)

