"""Whole-step graph capture (prlstm_amd.graph.GraphedTrainStep).

Each replay is compared with an eager forward+backward of the same module on the
same input, with eager work and synchronisations between replays (graph nodes
that only give correct results on the first replay would fail here).
"""

import pytest
import torch

import prlstm_amd
from prlstm_amd.graph import GraphedTrainStep

pytestmark = pytest.mark.gpu


def _eager(m, x):
    m.zero_grad(set_to_none=True)
    out, _ = m(x)
    out.sum().backward()
    return out.detach().clone(), {n: p.grad.detach().clone() for n, p in m.named_parameters() if p.grad is not None}


@pytest.mark.parametrize("parallel", [False, True])
@pytest.mark.parametrize("shape", [(16, 8, 32, 64), (256, 32, 256, 512)])
def test_graph_replays_match_eager(dev, parallel, shape):
    _check_replays(dev, parallel, shape)


def test_graph_replays_split_products(dev):
    """Parallel mode at a size whose input projection (1024 tiles of 256x256) and dW_ih
    (34 GFLOP in 8 k-splits summed in fp64) run on the split-bf16 kernels."""
    _check_replays(dev, True, (1024, 16, 256, 1024))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_graph_replays_half_module_parallel(dev, dtype):
    """A 16-bit module in parallel mode (16-bit projection, the scan storing out and reading
    dout in the module's format) replayed as one graph: every replay equals an eager step."""
    _check_replays(dev, True, (64, 8, 32, 64), dtype)


@pytest.mark.parametrize("parallel", [False, True])
def test_graph_replays_f64_module(dev, parallel):
    """An fp64 module (the *_f64 kernels, one launch per step in recurrent mode) replayed as
    one graph: every replay equals an eager step."""
    _check_replays(dev, parallel, (24, 4, 16, 32), torch.float64)


def _check_replays(dev, parallel, shape, dtype=torch.float32):
    T, B, D, H = shape
    print(f"graph T={T} B={B} D={D} H={H} parallel={parallel} dtype={dtype}", flush=True)
    torch.manual_seed(0)
    m = prlstm_amd.HeadStartLSTM(D, H, parallel=parallel).to(dev, dtype)
    with torch.no_grad():
        m.a.fill_(0.3)
    other = prlstm_amd.HeadStartLSTM(D, H).to(dev)
    x0 = torch.randn(T, B, D, device=dev).to(dtype)
    step = GraphedTrainStep(m, x0)
    for rep in range(4):
        x = torch.randn(T, B, D, device=dev).to(dtype)
        out_g = step.step(x).detach().clone()
        grads_g = {n: p.grad.detach().clone() for n, p in m.named_parameters() if p.grad is not None}
        torch.cuda.synchronize()
        # eager work in between, on the same stream
        _eager(other, torch.randn(T, B, D, device=dev))
        torch.cuda.synchronize()
        # eager reference on a clone of the module (the graph owns m's .grad tensors)
        ref = prlstm_amd.HeadStartLSTM(D, H, parallel=parallel).to(dev, dtype)
        ref.load_state_dict(m.state_dict())
        out_e, grads_e = _eager(ref, x)
        assert torch.allclose(out_g, out_e, rtol=1e-6, atol=1e-7), rep
        assert set(grads_g) == set(grads_e)
        for n in grads_e:
            assert torch.allclose(grads_g[n], grads_e[n], rtol=1e-5, atol=1e-6), (rep, n)


@pytest.mark.parametrize("shape", [(16, 8, 32, 64), (128, 32, 256, 256)])
def test_head_start_schedule_mode_switch(dev, shape):
    """The head-start schedule (README.md:13-16): parallel steps, then recurrent, then
    parallel again, with an SGD update after every step.  One GraphedTrainStep follows
    the module's mode (one graph per mode); an eager twin runs the same schedule.  After
    every step the outputs, the gradients (None where eager leaves None) and the updated
    parameters must agree."""
    T, B, D, H = shape
    print(f"schedule T={T} B={B} D={D} H={H}", flush=True)
    torch.manual_seed(1)
    m = prlstm_amd.HeadStartLSTM(D, H, parallel=True).to(dev)
    with torch.no_grad():
        m.a.fill_(0.2)
    twin = prlstm_amd.HeadStartLSTM(D, H, parallel=True).to(dev)
    twin.load_state_dict(m.state_dict())
    xs = [torch.randn(T, B, D, device=dev) for _ in range(6)]
    step = GraphedTrainStep(m, xs[0])
    lr = 1e-3
    schedule = [True, True, False, False, True, False]
    for i, (parallel, x) in enumerate(zip(schedule, xs)):
        m.set_mode(parallel)
        twin.set_mode(parallel)
        out_g = step.step(x).detach().clone()
        grads_g = {n: (None if p.grad is None else p.grad.detach().clone()) for n, p in m.named_parameters()}
        twin.zero_grad(set_to_none=True)
        out_e, _ = twin(x)
        out_e.sum().backward()
        assert torch.allclose(out_g, out_e, rtol=1e-5, atol=1e-6), i
        for n, p in twin.named_parameters():
            if p.grad is None:
                assert grads_g[n] is None, (i, n)
            else:
                assert grads_g[n] is not None, (i, n)
                assert torch.allclose(grads_g[n], p.grad, rtol=1e-4, atol=1e-5), (i, n)
        with torch.no_grad():
            for mod in (m, twin):
                for p in mod.parameters():
                    if p.grad is not None:
                        p.add_(p.grad, alpha=-lr)
        torch.cuda.synchronize()
    for (n, p), (_, q) in zip(m.named_parameters(), twin.named_parameters()):
        assert torch.allclose(p, q, rtol=1e-5, atol=1e-6), n
    assert set(step._graphs) == {True, False}
