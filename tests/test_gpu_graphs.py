"""HIP graph capture of the drop-in DDPM (torch.cuda.graph).

Every operator launches on the stream torch reports as current (the C-ABI
takes it as an argument) and takes its workspaces from torch's allocator, so
a forward -- and a forward plus backward -- can be captured once and
replayed.  Each replay is compared bit for bit with the eager result on the
same inputs (every kernel is deterministic: fixed-order split reductions, no
atomics), with new inputs copied in, eager work and synchronizations between
the replays.  The backward is captured from a given output gradient, so the
graph holds this library's kernels and torch's element-wise autograd work
only (no multi-block torch reductions).

Cases: the fused route at 64 channels (fp32 and bf16, a 40 x 56 map whose
fuse convolution splits its input-plane loop) and the materialized route at
K = 5 (bf16).
"""

import pytest
import torch

from dynamicconvolutionoperator_amd import DDPM
from tests.gpu_helpers import DEV, randn, say

pytestmark = pytest.mark.gpu

CASES = [(64, 3, 64, 64, torch.float32), (64, 3, 40, 56, torch.bfloat16), (24, 5, 16, 24, torch.bfloat16)]


def _module(c, k, dt):
    torch.manual_seed(31)
    return DDPM(c, k).to(DEV).to(dt)


def _fill(x, y, c, h, w, dt, seed):
    x.copy_(randn((1, c, h, w), seed).to(dt))
    y.copy_(randn((1, c, h, w), seed + 1).to(dt))


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"C{c[0]}K{c[1]}_{c[2]}x{c[3]}_{str(c[4])[6:]}")
def test_inference_graph_replays_match_eager(case):
    c, k, h, w, dt = case
    say(f"graph inference C={c} K={k} {h}x{w} {dt}")
    m = _module(c, k, dt).eval()
    x = torch.empty(1, c, h, w, device=DEV, dtype=dt)
    y = torch.empty_like(x)
    _fill(x, y, c, h, w, dt, 700)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.no_grad():
        with torch.cuda.stream(side):
            for _ in range(2):
                m(x, y)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = m(x, y)
        for i in range(3):
            _fill(x, y, c, h, w, dt, 710 + 2 * i)
            graph.replay()
            torch.cuda.synchronize()
            eager = m(x, y)
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {i}: max|diff| {(out.float() - eager.float()).abs().max().item():.3e}"


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"C{c[0]}K{c[1]}_{c[2]}x{c[3]}_{str(c[4])[6:]}")
def test_training_graph_replays_match_eager(case):
    c, k, h, w, dt = case
    say(f"graph forward+backward C={c} K={k} {h}x{w} {dt}")
    m = _module(c, k, dt).train()
    x = torch.empty(1, c, h, w, device=DEV, dtype=dt, requires_grad=True)
    y = torch.empty_like(x, requires_grad=True)
    gout = torch.empty(1, c, h, w, device=DEV, dtype=dt)
    with torch.no_grad():
        _fill(x, y, c, h, w, dt, 800)
        gout.copy_(randn((1, c, h, w), 799).to(dt))
    params = list(m.parameters())

    def step():
        torch.autograd.backward(m(x, y), gout)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            m.zero_grad(set_to_none=True)
            x.grad = None
            y.grad = None
            step()
    torch.cuda.current_stream().wait_stream(side)
    m.zero_grad(set_to_none=True)
    x.grad = None
    y.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    leaves = [x, y, *params]
    for i in range(3):
        with torch.no_grad():
            _fill(x, y, c, h, w, dt, 810 + 2 * i)
            gout.copy_(randn((1, c, h, w), 809 + 2 * i).to(dt))
        graph.replay()
        torch.cuda.synchronize()
        grads = [t.grad.clone() for t in leaves]
        eager = torch.autograd.grad(m(x, y), leaves, gout)
        torch.cuda.synchronize()
        names = ["dx", "dy"] + [n for n, _ in m.named_parameters()]
        for name, a, e in zip(names, grads, eager):
            assert torch.equal(a, e), f"replay {i} {name}: max|diff| {(a.float() - e.float()).abs().max().item():.3e}"
